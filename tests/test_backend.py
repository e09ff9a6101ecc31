"""Mi355xBackend behind the reference compiler's backend interface (CPU).

The reference's Compiler calls backend.generate(ctx) on its CompileContext
after its own passes (src/nnc_py/compiler.py:181-247, codegen/base.py:32-45).
These tests hand the backend a context shaped like the reference's - nodes in
a dict keyed by name with enum op types, TensorType-like tensors with
shape.dims and enum dtypes, constants in a separate dict (ir/graph.py:12-60,
node.py:95-124, tensor.py:9-53) - built here without importing the
reference, and check:
  * its files equal, byte for byte, what Compiler(target="mi355x").compile
    writes for the same graph (ResNet-18, LeNet-5, the transformer encoder,
    the bandwidth chain; O1 and O3; a memory budget; another entry name);
  * a graph as the reference's O3 passes leave it (pattern-fused nodes under
    the reference's names, FusedConvBiasRelu, transposed Gemm weights, the
    fused-away tensors still listed, nodes in another topological order)
    gives a program whose outputs on the oracle equal the unfused graph's
    bit for bit;
  * the result can be written the way the reference's Compiler writes it.
"""

from __future__ import annotations

import enum
from types import SimpleNamespace

import numpy as np
import pytest

import caserun


class RefDataType(enum.Enum):  # values of the reference's DataType
    FLOAT32 = "float32"
    FLOAT16 = "float16"
    INT32 = "int32"
    INT64 = "int64"
    INT8 = "int8"
    UINT8 = "uint8"
    BOOL = "bool"


def _op_enum(names):
    return enum.Enum("RefOpType", {n.upper(): n for n in sorted(names)})


class RefGraph:
    """nodes: dict name -> node; topological_sort() as the reference's
    (a valid order; here Kahn's algorithm, optionally newest-first)."""

    def __init__(self, name, lifo=False):
        self.name = name
        self.nodes, self.tensors, self.constants = {}, {}, {}
        self.inputs, self.outputs = [], []
        self.lifo = lifo

    def topological_sort(self):
        produced = {t: n for n in self.nodes.values() for t in n.outputs}
        deps = {n.name: {produced[t].name for t in n.inputs if t in produced} for n in self.nodes.values()}
        done, order = set(), []
        pending = list(self.nodes)
        while pending:
            ready = [n for n in pending if deps[n] <= done]
            pick = ready[-1] if self.lifo else ready[0]
            order.append(self.nodes[pick])
            done.add(pick)
            pending.remove(pick)
        return order


def ref_context(graph, opt_level, metadata=None, lifo=False):
    """A reference-shaped CompileContext holding `graph` (this package's IR)."""
    ops = _op_enum({n.op_type for n in graph.nodes} | {"FusedConvBiasRelu", "FusedConvRelu", "FusedAddRelu",
                                                       "FusedMatMulRelu"})
    rg = RefGraph(graph.name, lifo=lifo)
    for name, t in graph.tensors.items():
        rg.tensors[name] = SimpleNamespace(name=name, dtype=RefDataType(t.dtype),
                                           shape=SimpleNamespace(dims=list(t.shape), layout="nchw"))
        if t.is_constant:
            rg.constants[name] = t.data.copy()
    for n in graph.nodes:
        rg.nodes[n.name] = SimpleNamespace(op_type=ops(n.op_type), name=n.name, inputs=list(n.inputs),
                                           outputs=list(n.outputs), attrs=dict(n.attrs), metadata={})
    rg.inputs, rg.outputs = list(graph.inputs), list(graph.outputs)
    md = {"entry_point": "nnc_run"}
    md.update(metadata or {})
    return SimpleNamespace(graph=rg, target="mi355x", optimization_level=opt_level, debug=False, metadata=md,
                           tensor_symbols={}, node_symbols={}), ops


def _files(result):
    return {a.filename: (a.file_type, a.content) for a in result.files}


def _written(tmp_path, graph, opt, **kw):
    from nnc_py_amd.compiler.compiler import Compiler
    out = tmp_path / f"o{opt}"
    Compiler(target="mi355x", opt_level=opt).compile(graph, str(out), **kw)
    return {p.name: (p.read_bytes() if p.name.endswith(".bin") else p.read_text()) for p in out.iterdir()}


MODELS = {
    "resnet18": lambda z: z.resnet18(batch=1, seed=0),
    "lenet5": lambda z: z.lenet5(batch=2, seed=0),
    "transformer": lambda z: z.transformer_encoder(batch=1, seq=16, seed=0),
    "chain": lambda z: z.bandwidth_chain(batch=2, channels=8, hw=6, rows_softmax=4, len_softmax=16, rows_ln=4,
                                         len_ln=12, red_channels=4, red_hw=3),
}


@pytest.mark.parametrize("model", sorted(MODELS))
@pytest.mark.parametrize("opt", [1, 3])
def test_generate_equals_compile(model, opt, pkg, tmp_path):
    from nnc_py_amd.compiler import zoo
    from nnc_py_amd.compiler.backend import Mi355xBackend
    ctx, _ = ref_context(MODELS[model](zoo), opt)
    result = Mi355xBackend().generate(ctx)
    got = _files(result)
    want = _written(tmp_path, MODELS[model](zoo), opt)
    assert sorted(got) == sorted(want) == sorted(["model.h", "model.c", "tensors.c", "constants_loader.c",
                                                  "constants.bin", "test_runner.c", "Makefile"])
    for name, (kind, content) in got.items():
        assert (kind == "binary") == name.endswith(".bin")
        assert content == want[name], name
    assert result.metadata["target"] == "mi355x" and result.metadata["calls"] > 0


def test_generate_reads_entry_point_budget_and_strategy(pkg, tmp_path, monkeypatch):
    from nnc_py_amd.compiler import executor, zoo
    from nnc_py_amd.compiler.backend import Mi355xBackend
    # (with the residual Add fused into its LayerNorm this encoder's plan
    # peaks at the FFN MatMul's own working set, which no spill can lower:
    # the budget test runs on the unfused program, whose peak can)
    monkeypatch.setattr(executor, "ELTWISE_FUSION", False)
    g = zoo.transformer_encoder(batch=2, seq=16, seed=0)
    from nnc_py_amd.compiler import build_program
    peak = build_program(zoo.transformer_encoder(batch=2, seq=16, seed=0), 3).plan.activation_bytes
    budget = int(peak * 0.9)
    ctx, _ = ref_context(g, 3, {"entry_point": "encoder_run", "max_memory": budget,
                                "memory_strategy": "cost_aware"})
    backend = Mi355xBackend()
    got = _files(backend.generate(ctx))
    assert "encoder_run" in got["model.h"][1]
    assert backend.last_program.plan.slow_bytes > 0  # spilled to fit the budget
    assert backend.last_program.plan.activation_bytes <= budget
    want = _written(tmp_path, zoo.transformer_encoder(batch=2, seq=16, seed=0), 3, entry_point="encoder_run",
                    max_memory=str(budget), memory_strategy="cost_aware")
    assert all(got[k][1] == want[k] for k in want)
    bad, _ = ref_context(zoo.lenet5(), 1, {"memory_strategy": "greedy"})
    with pytest.raises(ValueError):
        backend.generate(bad)


def _reference_o3_shape(ctx, ops):
    """Rewrite the context's graph as the reference's O3 passes leave it:
    Conv+Relu / Add+Relu / MatMul+Relu pairs replaced by one fused node
    named fused_<pattern>_<n> appended to the node dict (pattern_fusion.py:
    63-135), the fused-away intermediate tensors still listed, the first
    fused conv as FusedConvBiasRelu, and constant Gemm weights transposed
    with transB = 1 (prepack_lowering.py:80-118)."""
    g = ctx.graph
    pairs = [("Conv", "Relu", "FusedConvRelu", "conv_relu"), ("Add", "Relu", "FusedAddRelu", "add_relu"),
             ("MatMul", "Relu", "FusedMatMulRelu", "matmul_relu")]
    count = 0
    for prod_op, cons_op, fused_op, tag in pairs:
        for name in list(g.nodes):
            n = g.nodes.get(name)
            if n is None or n.op_type.value != prod_op or n.outputs[0] in g.outputs:
                continue
            users = [u for u in g.nodes.values() if n.outputs[0] in u.inputs]
            if len(users) != 1 or users[0].op_type.value != cons_op:
                continue
            count += 1
            op = "FusedConvBiasRelu" if fused_op == "FusedConvRelu" and count == 1 else fused_op
            fused = SimpleNamespace(op_type=ops(op), name=f"fused_{tag}_{count}", inputs=list(n.inputs),
                                    outputs=list(users[0].outputs), attrs=dict(n.attrs),
                                    metadata={"fused_from": [n.name, users[0].name]})
            del g.nodes[n.name], g.nodes[users[0].name]
            g.nodes[fused.name] = fused
    for n in g.nodes.values():
        if n.op_type.value == "Gemm" and int(n.attrs.get("transB", 0)) == 0 and n.inputs[1] in g.constants:
            w = np.ascontiguousarray(g.constants[n.inputs[1]].T)
            g.constants[n.inputs[1]] = w
            g.tensors[n.inputs[1]].shape.dims = list(w.shape)
            n.attrs["transB"] = 1
    return count


def _run_on_oracle(prog, oracle_lib, feeds):
    from nnc_py_amd.compiler import Executor
    ex = Executor(prog, device=False, lib=oracle_lib)
    for k, v in feeds.items():
        ex.set_input(k, v)
    ex.run()
    return {o: ex.get(o) for o in prog.graph.outputs}


@pytest.mark.parametrize("model", ["lenet5", "resnet18", "transformer"])
@pytest.mark.parametrize("opt", [1, 3])
def test_reference_o3_graph_runs_like_the_original(model, opt, pkg, oracle_lib):
    from nnc_py_amd.compiler import build_program, zoo
    from nnc_py_amd.compiler.backend import Mi355xBackend
    make = {"lenet5": lambda: zoo.lenet5(batch=2, seed=3),
            "resnet18": lambda: zoo.resnet18(batch=1, seed=3),
            "transformer": lambda: zoo.transformer_encoder(batch=1, seq=16, heads=1, seed=3)}[model]
    ctx, ops = ref_context(make(), opt, lifo=True)
    assert _reference_o3_shape(ctx, ops) > 0
    backend = Mi355xBackend()
    backend.generate(ctx)
    prog = backend.last_program
    assert not any(n.op_type == "FusedConvBiasRelu" for n in prog.order)
    base = build_program(make(), opt)
    rng = np.random.default_rng(1)
    feeds = {n: rng.standard_normal(base.graph.tensors[n].shape).astype(np.float32) for n in base.graph.inputs}
    got = _run_on_oracle(prog, oracle_lib, feeds)
    want = _run_on_oracle(base, oracle_lib, feeds)
    for o in want:
        assert caserun.same_bits(got[o], want[o]), o


def test_result_writes_like_the_reference_compiler(pkg, tmp_path):
    """The reference's Compiler._write_output (compiler.py:291-312): write
    each artifact by file_type, then set metadata entries."""
    from nnc_py_amd.compiler import zoo
    from nnc_py_amd.compiler.backend import Mi355xBackend
    ctx, _ = ref_context(zoo.lenet5(), 1)
    artifacts = Mi355xBackend().generate(ctx)
    for artifact in artifacts.files:
        path = tmp_path / artifact.filename
        if artifact.file_type == "binary":
            path.write_bytes(artifact.content)
        else:
            path.write_text(artifact.content)
    artifacts.metadata["entry_point"] = "nnc_run"
    artifacts.metadata["target"] = "mi355x"
    artifacts.metadata["opt_level"] = 1
    assert (tmp_path / "constants.bin").read_bytes()[:4] == b"NNCB"
    assert "nnc_run" in (tmp_path / "model.h").read_text()
