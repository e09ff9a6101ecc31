"""Compiler passes, arena plan and lowering (CPU only).

The O1 lowering of ResNet-18 and LeNet-5 must reproduce the call sequence of
the reference's codegen snapshots (tests/golden/snapshot_calls.json, extracted
from tests/__snapshots__/test_snapshots_{resnet18,lenet5}.ambr): same node
functions, entry points, activation tensors and integer/float arguments.
Constant tensor names differ (the reference's onnxsim renames folded
weights), so constants are compared by role only.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import caserun

GOLDEN = Path(__file__).resolve().parent / "golden" / "snapshot_calls.json"


def _lowered_calls(graph, opt):
    from nnc_py_amd.compiler import build_program
    from nnc_py_amd.compiler.codegen import Symbols
    prog = build_program(graph, opt_level=opt)
    syms = Symbols()
    for n in prog.graph.tensors:
        syms.get("tensor", n)
    out = []
    for c in prog.calls:
        args = []
        for a in c.args:
            if a[0] == "t":
                args.append(("const" if prog.graph.tensors[a[1]].is_constant else syms.get("tensor", a[1])))
            elif a[0] == "null":
                args.append(None)
            else:
                args.append(a[1])
        out.append({"node": syms.get("node", c.node), "op": c.op, "args": args})
    return prog, out


@pytest.mark.parametrize("model", ["resnet18", "lenet5"])
def test_o1_call_sequence_matches_reference_snapshot(model, pkg):
    from nnc_py_amd.compiler import zoo
    want = json.loads(GOLDEN.read_text())[model]
    graph = zoo.resnet18(batch=1, seed=0) if model == "resnet18" else zoo.lenet5(batch=1, seed=0)
    consts = set(graph.constants)
    prog, got = _lowered_calls(graph, 1)
    assert len(got) == len(want)
    for g, w in zip(got, want):
        assert g["node"] == w["node"], (g, w)
        assert g["op"] == w["op"], (g, w)
        assert len(g["args"]) == len(w["args"]), (g, w)
        for ga, wa in zip(g["args"], w["args"]):
            if ga == "const":
                assert isinstance(wa, str) and wa.startswith("tensor_")
            else:
                assert ga == wa, (g["node"], ga, wa)


def test_o3_fusion_and_prepack_on_resnet18(pkg):
    """O3: conv+relu fusion, each residual block's conv+add+relu as one call
    (in place only over the residual), every 3x3 conv with Ci % 32 == 0 on
    tap-major packed weights, conv entry selection for the rest, constant FC
    weight as gemm_nt."""
    from nnc_py_amd.compiler import build_program, zoo
    prog = build_program(zoo.resnet18(batch=2, seed=0), opt_level=3)
    ops = [c.op for c in prog.calls if c.node]  # without the stream fork/select/join calls
    assert len(ops) == 20  # Flatten is an alias of the pooled tensor: no call
    assert "nnc_flatten" not in ops and prog.plan.aliases
    assert ops.count("nnc_hip_conv_packed") == 14  # the stem and every 3x3 conv without a projection
    assert "nnc_add_relu" not in ops and "nnc_relu" not in ops
    # the three downsample blocks: their 1x1 projection folded into the last conv
    assert ops[0] == "nnc_hip_conv_packed" and ops.count("nnc_conv1x1") == 0 and ops.count("nnc_hip_conv_proj") == 3
    assert ops[-1] == "nnc_gemm_nt"
    with_res = [c for c in prog.calls if c.op == "nnc_hip_conv_packed" and c.args[3][0] == "t"]
    assert len(with_res) == 5
    for c in prog.calls:
        if c.op == "nnc_hip_conv_proj":
            h, w, x, out = (prog.graph.tensors[c.args[k][1]] for k in (0, 1, 3, 4))
            co, ci, cx = out.shape[1], h.shape[1], x.shape[1]
            assert w.shape == (co, 9 * ci + cx) and cx == ci // 2 and x.shape[2] == 2 * out.shape[2]
            assert [a[1] for a in c.args[5:]] == [3, 3, 1, 1, 1, 1, 2, 2, 1]
    for c in prog.calls:
        if c.op != "nnc_hip_conv_packed":
            continue
        assert c.args[-1] == ("i", 1)  # relu after every conv of ResNet-18 but the 1x1
        w = prog.graph.tensors[c.args[1][1]]
        if c.args[5] == ("i", 7):
            assert w.shape == (64, 160)  # [Co][Kp]: 7*7*3 = 147 padded to 160
        else:
            assert w.shape[1:3] == (3, 3) and w.shape[3] % 32 == 0  # [Co][kh][kw][Ci]
        if c.args[3][0] == "t":
            res, out = c.args[3][1], c.args[4][1]
            assert prog.graph.tensors[res].shape == prog.graph.tensors[out].shape
            assert prog.plan.offsets[out] != prog.plan.offsets[c.args[0][1]]


def test_packed_conv_weights_are_the_transposed_constants(pkg):
    from nnc_py_amd.compiler import build_program, zoo
    ref = zoo.resnet18(batch=1, seed=0)
    orig = {k: t.data.copy() for k, t in ref.tensors.items() if t.is_constant and t.data is not None
            and t.data.ndim == 4}
    prog = build_program(ref, opt_level=3)
    n = 0
    for c in prog.calls:
        if c.op == "nnc_hip_conv_packed":
            name = c.args[1][1]
            packed, w = prog.graph.tensors[name].data, orig[name]
            if packed.ndim == 2:  # [Co][Kp]: tap-major rows, zero past K
                k = w[0].size
                np.testing.assert_array_equal(packed[:, :k], w.transpose(0, 2, 3, 1).reshape(w.shape[0], k))
                assert not packed[:, k:].any() and packed.shape[1] % 32 == 0
            else:
                np.testing.assert_array_equal(packed, w.transpose(0, 2, 3, 1))
            n += 1
        elif c.op == "nnc_hip_conv_proj":
            rows = prog.graph.tensors[c.args[1][1]].data
            node = next(m for m in prog.order if m.name == c.node)
            w3, w1 = (orig[m] for m in node.metadata["weights_from"])
            co = w3.shape[0]
            np.testing.assert_array_equal(rows, np.concatenate([w3.transpose(0, 2, 3, 1).reshape(co, -1),
                                                                w1.reshape(co, -1)], axis=1))
            n += 1
    assert n == 17


def test_target_rewrites_can_be_switched_off(pkg):
    """Without weight packing the residual blocks use nnc_hip_conv_add_relu;
    without residual fusion either, conv and add_relu are separate calls;
    target_passes=False gives the reference's own O3 call sequence."""
    from nnc_py_amd.compiler import build_program, zoo
    from nnc_py_amd.compiler import executor as ex_mod
    ex_mod.PACK_CONV_WEIGHTS = False
    try:
        prog = build_program(zoo.resnet18(batch=2, seed=0), opt_level=3)
        ops = [c.op for c in prog.calls if c.node]  # without stream fork/select/join
        assert len(ops) == 23 and ops.count("nnc_hip_conv_add_relu") == 8
        assert ops.count("nnc_conv_relu3x3_s1") == 5  # conv1 of the five stride-1 blocks
        assert ops[0] == "nnc_conv_relu7x7_s2"
        ex_mod.RESIDUAL_FUSION = False
        prog = build_program(zoo.resnet18(batch=2, seed=0), opt_level=3)
        ops = [c.op for c in prog.calls if c.node]
        assert len(ops) == 31 and ops.count("nnc_add_relu") == 8
    finally:
        ex_mod.PACK_CONV_WEIGHTS = True
        ex_mod.RESIDUAL_FUSION = True
    ops = [c.op for c in build_program(zoo.resnet18(batch=2, seed=0), opt_level=3, target_passes=False).calls]
    assert len(ops) == 32 and ops.count("nnc_add_relu") == 8 and "nnc_flatten" in ops
    assert not any(o.startswith("nnc_hip_") for o in ops)


def test_arena_plan_reuses_memory_and_keeps_invariants(pkg):
    from nnc_py_amd.compiler import build_program, zoo
    from nnc_py_amd.compiler.passes import check_plan
    basic = build_program(zoo.resnet18(batch=4, seed=0), opt_level=0)
    aware = build_program(zoo.resnet18(batch=4, seed=0), opt_level=1)
    check_plan(aware.graph, aware.order, aware.plan)
    assert aware.plan.activation_bytes < basic.plan.activation_bytes / 3
    assert aware.plan.inplace  # element-wise outputs written over dying inputs
    for out, inp in aware.plan.inplace.items():
        assert aware.plan.offsets[out] == aware.plan.offsets[inp]
    with pytest.raises(ValueError):
        build_program(zoo.resnet18(batch=4, seed=0), opt_level=1, max_memory=1 << 20)


def test_identity_and_dead_code_elimination(pkg):
    from nnc_py_amd.compiler import GraphBuilder, build_program
    b = GraphBuilder()
    x = b.input("x", (2, 8))
    y = b.identity(x)
    z = b.relu(y)
    b.sigmoid(x)  # dead
    b.output(b.tanh(z))
    prog = build_program(b.build(), opt_level=1)
    assert [c.op for c in prog.calls] == ["nnc_relu", "nnc_tanh"]
    assert prog.calls[0].args[0] == ("t", "x")


def test_multi_axis_reduce_lowers_to_a_merged_view(pkg):
    from nnc_py_amd.compiler import GraphBuilder, build_program
    b = GraphBuilder()
    x = b.input("x", (2, 4, 5, 6))
    b.output(b.reducemean(x, axes=(2, 3), keepdims=1))
    prog = build_program(b.build(), opt_level=1)
    (call,) = prog.calls
    assert call.op == "nnc_reducemean"
    assert call.args[0] == ("tv", "x", (2, 4, 30)) and call.args[2] == ("i", 2)


def test_executor_on_oracle_matches_numpy_for_reduce_chain(pkg, oracle_lib):
    from nnc_py_amd.compiler import Executor, GraphBuilder, build_program
    b = GraphBuilder()
    x = b.input("x", (3, 8, 7, 7))
    m = b.reducemean(x, axes=(2, 3), keepdims=1)
    b.output(b.reducesum(m, axes=(1,), keepdims=0))
    ex = Executor(build_program(b.build(), opt_level=1), device=False, lib=oracle_lib)
    v = np.random.default_rng(0).standard_normal((3, 8, 7, 7)).astype(np.float32)
    ex.set_input("x", v)
    ex.run()
    out = ex.get(b.g.outputs[0])
    np.testing.assert_allclose(out.ravel(), v.astype(np.float64).mean((2, 3)).sum(1), rtol=1e-5, atol=1e-5)


def test_o3_downsample_branches_on_the_second_stream(pkg):
    """Small batches: each downsample block's two convolutions reading the
    block input run on two streams (fork before the first, side call on
    stream 1, join before the residual conv); none of the tensors they touch
    is freed or reused before the join. Batch 32: every convolution fills
    the GPU alone, no branches."""
    from nnc_py_amd.compiler import build_program, zoo
    from nnc_py_amd.compiler.passes import check_plan, liveness
    assert not build_program(zoo.resnet18(batch=1, seed=0), opt_level=3).branches  # opt-in
    prog = build_program(zoo.resnet18(batch=1, seed=0), opt_level=3, branch_streams=True)
    assert len(prog.branches) == 3
    seq = [c.op for c in prog.calls]
    for i, op in enumerate(seq):
        if op == "nnc_hip_stream_fork":
            assert seq[i + 1:i + 4] == ["nnc_hip_stream_select", "nnc_hip_conv_packed", "nnc_hip_stream_select"]
            assert [a[1] for a in prog.calls[i + 1].args] == [1] and [a[1] for a in prog.calls[i + 3].args] == [0]
            assert seq[i + 4] == "nnc_conv1x1" and seq[i + 5] == "nnc_hip_stream_join"
            assert prog.calls[i + 6].op == "nnc_hip_conv_packed" and prog.calls[i + 6].args[3][0] == "t"
    assert seq.count("nnc_hip_stream_fork") == seq.count("nnc_hip_stream_join") == 3
    # every tensor of a concurrent pair stays live (unshared) until the join
    pos = {n.name: i for i, n in enumerate(prog.order)}
    live = liveness(prog.graph, prog.order, [[b.side] + b.main for b in prog.branches])
    for b in prog.branches:
        nodes = [prog.order[pos[n]] for n in [b.side] + b.main]
        end = max(pos[n.name] for n in nodes)
        touched = {t for n in nodes for t in list(n.inputs) + list(n.outputs) if t in live}
        assert all(live[t].end >= end for t in touched)
        offs = {t: prog.plan.offsets[t] for t in touched if t not in prog.graph.constants}
        sizes = {t: prog.graph.tensors[t].nbytes for t in offs}
        names = sorted(offs)
        for x in range(len(names)):
            for y in range(x + 1, len(names)):
                a, c = names[x], names[y]
                assert offs[a] + sizes[a] <= offs[c] or offs[c] + sizes[c] <= offs[a], (a, c)
    check_plan(prog.graph, prog.order, prog.plan, [[b.side] + b.main for b in prog.branches])
    assert not build_program(zoo.resnet18(batch=32, seed=0), opt_level=3, branch_streams=True).branches


def _self_residual_graph(batch=1, c=64, hw=16, seed=0):
    """relu(conv(h) + h) with h an intermediate: the fused conv reads h as
    its image and as its residual."""
    from nnc_py_amd.compiler import GraphBuilder
    rng = np.random.default_rng(seed)
    b = GraphBuilder("self_residual")
    x = b.input("x", (batch, c, hw, hw))

    def conv(t, name):
        w = b.const(f"{name}.w", (rng.standard_normal((c, c, 3, 3)) * np.sqrt(2.0 / (9 * c))).astype(np.float32))
        bias = b.const(f"{name}.b", (rng.standard_normal(c) * 0.01).astype(np.float32))
        return b.conv(t, w, bias, pads=(1, 1, 1, 1), name=f"/{name}")

    h = b.relu(conv(x, "c0"))
    s = b.add(conv(h, "c1"), h)
    b.output(b.relu(s))
    return b.build()


def test_fused_conv_never_writes_over_its_own_image(pkg):
    """relu(conv(h) + h): the residual is also the conv's image, which other
    workgroups still read while finished tiles are stored, so the output must
    not take over h's arena slot."""
    from nnc_py_amd.compiler import build_program
    from nnc_py_amd.compiler.passes import check_plan
    prog = build_program(_self_residual_graph(), opt_level=3)
    fused = [n for n in prog.order if n.op_type == "FusedConvAddRelu"]
    assert len(fused) == 1 and fused[0].inputs[0] == fused[0].inputs[3]
    h, out = fused[0].inputs[0], fused[0].outputs[0]
    assert out not in prog.plan.inplace
    assert prog.plan.offsets[out] != prog.plan.offsets[h]
    check_plan(prog.graph, prog.order, prog.plan)
    # a residual that is not the image may still be taken over
    from nnc_py_amd.compiler import zoo
    r18 = build_program(zoo.resnet18(batch=1, seed=0), opt_level=3)
    assert any(n.op_type in ("FusedConvAddRelu",) and n.outputs[0] in r18.plan.inplace for n in r18.order)


def test_gap_gemm_tile_streaming_pass(pkg):
    """stream_tiles at a batch it is allowed for: GlobalAveragePool ->
    Flatten -> Gemm(transB) becomes one FusedGapGemm lowered to
    nnc_hip_gap_gemm_nt, the pooled tensors gone, the decision and its LDS
    footprint in the node's metadata; above the batch limit, or over the LDS
    budget, the pair stays."""
    from nnc_py_amd.compiler import build_program, passes, zoo
    old = passes.GAP_GEMM_MAX_BATCH
    passes.GAP_GEMM_MAX_BATCH = 2
    try:
        prog = build_program(zoo.resnet18(batch=2, seed=0), opt_level=3)
        ops = [c.op for c in prog.calls]
        assert ops[-1] == "nnc_hip_gap_gemm_nt" and "nnc_avgpool2d" not in ops and len(ops) == 19
        node = next(n for n in prog.order if n.op_type == "FusedGapGemm")
        ts = node.metadata["tile_stream"]
        assert ts["lds_bytes"] == 4 * (512 + 512 * 50) <= ts["budget"] and ts["hbm_bytes_saved"] == 2 * 2 * 512 * 4
        assert prog.calls[-1].args[4:] == [("f", 1.0), ("f", 1.0)]
        big = [c.op for c in build_program(zoo.resnet18(batch=4, seed=0), opt_level=3).calls]
        assert big[-2:] == ["nnc_avgpool2d", "nnc_gemm_nt"]
        g = zoo.resnet18(batch=2, seed=0)
        assert passes.stream_tiles(g, lds_budget=4 * 512 * 50) == 0  # over the budget
    finally:
        passes.GAP_GEMM_MAX_BATCH = old


def test_conv_pool_tile_streaming_pass(pkg, oracle_lib):
    """stream_tiles with the stem fusion allowed: the packed stem conv +
    relu and its 3x3 / s2 / p1 max pool become one FusedConvMaxPool lowered
    to nnc_hip_conv_maxpool (the 112 x 112 activation gone); on the oracle
    the program computes the unfused program's bits (the same conv, relu and
    max). Below the batch limit, or by default, the pair stays."""
    from nnc_py_amd.compiler import Executor, build_program, passes, zoo
    assert build_program(zoo.resnet18(batch=2, seed=0), opt_level=3).calls[0].op == "nnc_hip_conv_packed"
    old = passes.CONV_POOL_MIN_ROWS
    passes.CONV_POOL_MIN_ROWS = 224  # batch 2 of 112 conv rows, not batch 1
    try:
        prog = build_program(zoo.resnet18(batch=2, seed=0), opt_level=3)
        small = build_program(zoo.resnet18(batch=1, seed=0), opt_level=3)
    finally:
        passes.CONV_POOL_MIN_ROWS = old
    ops = [c.op for c in prog.calls]
    assert ops[0] == "nnc_hip_conv_maxpool" and "nnc_maxpool2d" not in ops and len(ops) == 19
    assert [a[1] for a in prog.calls[0].args[4:]] == [7, 7, 2, 2, 3, 3]
    node = prog.order[0]
    assert node.op_type == "FusedConvMaxPool" and node.metadata["tile_stream"]["hbm_bytes_saved"] == 2 * 2 * 64 * 112 * 112 * 4
    assert small.calls[0].op == "nnc_hip_conv_packed"
    x = np.random.default_rng(4).standard_normal((2, 3, 224, 224)).astype(np.float32)
    outs = []
    for p in (prog, build_program(zoo.resnet18(batch=2, seed=0), opt_level=3)):
        ex = Executor(p, device=False, lib=oracle_lib)
        ex.set_input("input", x)
        ex.run()
        outs.append(ex.get("output"))
    assert outs[0].tobytes() == outs[1].tobytes()


_BW_SMALL = dict(batch=2, channels=8, hw=6, rows_softmax=4, len_softmax=16, rows_ln=4, len_ln=8, red_channels=4,
                 red_hw=4)


def test_eltwise_chains_of_the_bandwidth_chain(pkg, oracle_lib):
    """O3 (mi355x target): the bandwidth chain's element-wise ops become two
    FusedEltwise nodes - tanh(x - y), then relu(x + y) * x, clip(-6, 6),
    sigmoid, plus that tanh - lowered to nnc_hip_fused_eltwise, and its
    Concat -> Split round trip is gone. On the oracle every output has the
    bits of the reference pipeline's O3 program."""
    from nnc_py_amd.compiler import Executor, build_program, zoo
    prog = build_program(zoo.bandwidth_chain(**_BW_SMALL), opt_level=3)
    ops = [n.op_type for n in prog.order]
    assert ops.count("FusedEltwise") == 2
    assert not {"Concat", "Split", "Mul", "Clip", "Sigmoid", "Tanh", "Sub", "FusedAddRelu", "Add"} & set(ops)
    tanh_node, main = [n for n in prog.order if n.op_type == "FusedEltwise"]
    assert tanh_node.inputs == ["x", "y"] and tanh_node.attrs["steps"] == [[1, 0, 1, 0.0, 0.0], [8, -1, -1, 0.0, 0.0]]
    assert main.inputs == ["x", "y", tanh_node.outputs[0]] and main.outputs == ["chain"]
    assert [s[:3] for s in main.attrs["steps"]] == [[4, 0, 1], [2, -1, 0], [9, -1, -1], [7, -1, -1], [0, -1, 2]]
    assert main.attrs["steps"][2][3:] == [-6.0, 6.0]
    assert main.metadata["fused_from"] == ["/Add", "/Mul", "/Clip", "/Sigmoid", "/Add_1"]
    calls = [c.op for c in prog.calls]
    assert calls.count("nnc_hip_fused_eltwise") == 2 and "nnc_concat" not in calls and "nnc_split" not in calls
    ref = build_program(zoo.bandwidth_chain(**_BW_SMALL), opt_level=3, target_passes=False)
    assert "nnc_hip_fused_eltwise" not in [c.op for c in ref.calls] and "nnc_concat" in [c.op for c in ref.calls]
    rng = np.random.default_rng(8)
    feeds = {n: (rng.standard_normal(prog.graph.tensors[n].shape) * 4).astype(np.float32)
             for n in ("x", "y", "s", "l", "r")}
    outs = []
    for p in (prog, ref):
        ex = Executor(p, device=False, lib=oracle_lib)
        for k, v in feeds.items():
            ex.set_input(k, v)
        ex.run()
        outs.append({o: ex.get(o) for o in ("chain", "softmax", "layernorm", "mean", "sum")})
    for o in outs[0]:
        assert outs[0][o].tobytes() == outs[1][o].tobytes(), o


def test_eltwise_chain_limits(pkg):
    """A chain holds at most EW_MAX_STEPS nodes and EW_MAX_INPUTS distinct
    inputs, and ends at an output read twice, at a graph output and before
    a broadcast operand; a lone node stays as it is."""
    from nnc_py_amd.compiler import GraphBuilder, build_program, passes

    def fused(build):
        b = GraphBuilder("chains")
        build(b)
        return [(n.op_type, len(n.attrs.get("steps", []))) for n in build_program(b.build(), opt_level=3).order]

    def long_chain(b):
        t = b.input("x", (4, 8))
        for i in range(passes.EW_MAX_STEPS + 2):
            t = b.sigmoid(t, name=f"/s{i}")
        b.output(t)
    assert fused(long_chain) == [("FusedEltwise", passes.EW_MAX_STEPS), ("FusedEltwise", 2)]

    def five_inputs(b):
        xs = [b.input(f"x{i}", (4, 8)) for i in range(5)]
        t = b.add(xs[0], xs[1])
        for x in xs[2:]:
            t = b.add(t, x)
        b.output(t)
    assert fused(five_inputs) == [("FusedEltwise", 3), ("Add", 0)]

    def fan_out(b):
        u = b.relu(b.input("x", (4, 8)))
        b.output(b.sigmoid(u))
        b.output(b.tanh(u))
    assert sorted(fused(fan_out)) == [("Relu", 0), ("Sigmoid", 0), ("Tanh", 0)]

    def output_inside(b):
        u = b.relu(b.input("x", (4, 8)))
        b.output(u)
        b.output(b.sigmoid(u))
    assert sorted(fused(output_inside)) == [("Relu", 0), ("Sigmoid", 0)]

    def broadcast(b):
        bias = b.input("bias", (8,))
        b.output(b.sigmoid(b.tanh(b.add(b.input("x", (4, 8)), bias))))
    assert fused(broadcast) == [("Add", 0), ("FusedEltwise", 2)]


def test_transformer_add_layernorm_and_transposes(pkg, oracle_lib, monkeypatch):
    """O3 (mi355x target) on the transformer encoder: each residual Add and
    the LayerNormalization reading it become one FusedAddLayerNorm
    (nnc_hip_add_layernorm), each score scaling Div and its Softmax become
    one ScaledSoftmax (nnc_hip_scaled_softmax), K's head transpose
    followed by its transpose for Q K^T becomes one Transpose ([0,2,1,3]
    then [0,1,3,2] = [0,2,3,1]), and the QKV Split's pieces are transposed
    straight from the projection's output (nnc_hip_transpose_slice): 36 ->
    26 calls. On the oracle the output has the bits of the
    same O3 program without these rewrites."""
    from nnc_py_amd.compiler import Executor, build_program, executor, zoo
    kw = dict(batch=2, seq=8, d_model=16, heads=2, ffn=32, seed=3)
    prog = build_program(zoo.transformer_encoder(**kw), opt_level=3)
    ops = [c.op for c in prog.calls]
    assert ops.count("nnc_hip_add_layernorm") == 4 and "nnc_layernorm" not in ops and "nnc_add" not in ops
    assert ops.count("nnc_hip_scaled_softmax") == 2 and "nnc_softmax" not in ops and "nnc_div" not in ops
    assert ops.count("nnc_hip_transpose_slice") == 6 and "nnc_split" not in ops
    perms = [c.args[2][1] for c in prog.calls if c.op in ("nnc_transpose", "nnc_hip_transpose_slice")]
    assert perms.count([0, 2, 3, 1]) == 2 and [0, 1, 3, 2] not in perms
    monkeypatch.setattr(executor, "ATTENTION_FUSION", False)
    assert len(build_program(zoo.transformer_encoder(seed=1), opt_level=3).calls) == 26
    monkeypatch.setattr(executor, "ELTWISE_FUSION", False)
    ref = build_program(zoo.transformer_encoder(**kw), opt_level=3)
    assert [c.op for c in ref.calls].count("nnc_layernorm") == 4 and len(ref.calls) == len(prog.calls) + 10
    x = (np.random.default_rng(5).standard_normal((2, 8, 16)) * 0.5).astype(np.float32)
    outs = []
    for p in (prog, ref):
        ex = Executor(p, device=False, lib=oracle_lib)
        ex.set_input("input", x)
        ex.run()
        outs.append(ex.get(p.graph.outputs[0]))
    assert outs[0].tobytes() == outs[1].tobytes()


def test_transformer_attention_fusion(pkg, oracle_lib, monkeypatch):
    """O3 (mi355x target) on the transformer encoder: each layer's attention
    block - the head split transposes of Q, K^T and V, Q K^T, the scaled
    softmax, the product with V and the head merge - becomes one Attention
    node (nnc_hip_attention) reading the QKV projection's output and
    writing the merged heads the output projection reads: 26 -> 14 calls at
    batch 8, sequence 128. On the oracle, with one batch and one head (where
    the reference's batched MatMul stepping is the model's arithmetic), the
    output has the bits of the same O3 program without the fusion; with
    four heads (four attention batches, which the unfused program's
    reference-stepped MatMul gets wrong) it is within the fp bar of the
    float64 model.
    Heads of 16 or sequences that are no multiple of 32 are left alone."""
    from nnc_py_amd.compiler import Executor, build_program, executor, zoo
    prog = build_program(zoo.transformer_encoder(seed=1), opt_level=3)
    ops = [c.op for c in prog.calls]
    assert len(ops) == 14 and ops.count("nnc_hip_attention") == 2
    assert not {"nnc_hip_transpose_slice", "nnc_matmul", "nnc_hip_scaled_softmax", "nnc_transpose"} & set(ops)
    att = next(c for c in prog.calls if c.op == "nnc_hip_attention")
    assert [a[1] for a in att.args[3:]] == [8, 128, 4, 64, 0, 256, 512]
    assert att.args[0][1].endswith("qkv/Add_output")
    out_proj = prog.calls[ops.index("nnc_hip_attention") + 1]
    # the output projection reads the merged heads through the Reshape's view (same arena offset)
    assert out_proj.op == "nnc_gemm_nt"
    assert prog.plan.offsets[out_proj.args[0][1]] == prog.plan.offsets[att.args[2][1]]

    kw = dict(batch=1, seq=32, d_model=64, heads=1, ffn=128, seed=4)
    fused = build_program(zoo.transformer_encoder(**kw), opt_level=3)
    assert [c.op for c in fused.calls].count("nnc_hip_attention") == 2
    monkeypatch.setattr(executor, "ATTENTION_FUSION", False)
    plain = build_program(zoo.transformer_encoder(**kw), opt_level=3)
    assert "nnc_hip_attention" not in [c.op for c in plain.calls]
    monkeypatch.setattr(executor, "ATTENTION_FUSION", True)
    x = (np.random.default_rng(6).standard_normal((1, 32, 64)) * 0.5).astype(np.float32)
    outs = []
    for p in (fused, plain):
        ex = Executor(p, device=False, lib=oracle_lib)
        ex.set_input("input", x)
        ex.run()
        outs.append(ex.get(p.graph.outputs[0]))
    assert outs[0].tobytes() == outs[1].tobytes()

    kw = dict(batch=1, seq=64, d_model=128, heads=4, ffn=256, seed=5)
    multi = build_program(zoo.transformer_encoder(**kw), opt_level=3)
    assert [c.op for c in multi.calls].count("nnc_hip_attention") == 2
    x = (np.random.default_rng(7).standard_normal((1, 64, 128)) * 0.5).astype(np.float32)
    ex = Executor(multi, device=False, lib=oracle_lib)
    ex.set_input("input", x)
    ex.run()
    ref = zoo.transformer_encoder_reference(zoo.transformer_encoder(**kw), x, heads=4)
    assert caserun.fp_violations(ex.get("output"), ref, 1e-4, 1e-3).size == 0

    for kw in (dict(batch=1, seq=32, d_model=64, heads=4, ffn=64), dict(batch=1, seq=48, d_model=64, heads=1, ffn=64)):
        ops = [c.op for c in build_program(zoo.transformer_encoder(**kw), opt_level=3).calls]
        assert "nnc_hip_attention" not in ops and "nnc_matmul" in ops
