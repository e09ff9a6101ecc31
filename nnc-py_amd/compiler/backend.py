"""The mi355x target as a backend of the reference compiler.

The reference's Compiler runs its pass pipeline on a CompileContext and then
calls ``self.backend.generate(ctx)``; the result must carry ``files`` (each
with ``filename``, ``content``, ``file_type``), which it writes, and a
``metadata`` dict, which it updates (src/nnc_py/compiler.py:181-247, 266-285,
291-312; codegen/base.py:11-45). ``Mi355xBackend`` is that backend for the
MI355X: ``Compiler._create_backend("mi355x")`` returns it, and
``generate(ctx)`` returns the same artifact set as this package's
``Compiler(target="mi355x").compile`` writes for the same graph.

What it reads from a reference-shaped context (no import of the reference
package: attributes only, src/nnc_py/ir/context.py:26-49, graph.py:12-60,
node.py:95-124, tensor.py:9-53):

  ctx.graph.nodes        dict name -> node (or a list): op_type (an enum
                         whose .value is the op string, or the string),
                         name, inputs, outputs, attrs
  ctx.graph.tensors      dict name -> tensor: dtype (enum .value or str),
                         shape.dims (or shape)
  ctx.graph.constants    dict name -> numpy array
  ctx.graph.inputs/outputs
  ctx.optimization_level, ctx.debug
  ctx.metadata           entry_point, max_memory (bytes), memory_strategy

The reference's own passes have already run on that graph: its pattern
fusion leaves FusedConvRelu / FusedConvBiasRelu / FusedConvSigmoid /
FusedAddRelu / FusedAddSigmoid / FusedMatMulRelu nodes, its prepack pass
transposes constant Gemm weights and sets transB (prepack_lowering.py:80-118).
Both are ordinary graph semantics here. Their schedule and memory plan
(liveness, tiling, joint solution in ctx.metadata) are x86 decisions and
are not used: the backend plans the graph again with the mi355x passes,
the HBM arena planner and the lowering of this package (build_program).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np

from . import codegen
from .executor import Program, build_program
from .ir import Graph, Node, TensorInfo

REPO_ROOT = Path(__file__).resolve().parents[2]

# reference op strings that name the same arithmetic as one of ours
# (c_emitter.py:945-972 lowers FusedConvBiasRelu exactly as FusedConvRelu)
_OP_ALIASES = {"FusedConvBiasRelu": "FusedConvRelu"}


@dataclass
class CodeArtifact:
    """One generated file (the reference's codegen/base.py:11-17)."""
    filename: str
    content: str | bytes
    file_type: str = "source"  # "source", "header", "build" or "binary"


@dataclass
class CodeGenResult:
    """Generated files plus metadata (the reference's codegen/base.py:20-29)."""
    files: list[CodeArtifact] = field(default_factory=list)
    metadata: dict[str, Any] = field(default_factory=dict)

    def add_file(self, filename: str, content: str | bytes, file_type: str = "source") -> None:
        self.files.append(CodeArtifact(filename, content, file_type))


@dataclass
class CompileContext:
    """The fields of the reference's CompileContext this backend reads; this
    package's Compiler builds one around a Graph of its own."""
    graph: Any
    target: str = "mi355x"
    optimization_level: int = 0
    debug: bool = False
    metadata: dict[str, Any] = field(default_factory=dict)


def _value(v) -> Any:
    """An enum member's value, or the object itself."""
    return getattr(v, "value", v)


def _dims(t) -> tuple:
    shape = getattr(t, "shape", ())
    dims = getattr(shape, "dims", shape)
    out = []
    for d in dims:
        if not isinstance(d, (int, np.integer)):
            raise ValueError(f"tensor {getattr(t, 'name', '?')!r} has a symbolic dimension {d!r}: "
                             "the mi355x target needs static shapes")
        out.append(int(d))
    return tuple(out)


def _ordered_nodes(rg) -> list:
    nodes = rg.nodes
    if hasattr(rg, "topological_sort"):
        return list(rg.topological_sort())
    return list(nodes.values()) if isinstance(nodes, dict) else list(nodes)


def graph_from_context(ctx) -> Graph:
    """This package's Graph from ctx.graph: the reference IR (by attribute) or
    already a Graph (returned as is)."""
    rg = ctx.graph
    if isinstance(rg, Graph):
        return rg
    g = Graph(str(getattr(rg, "name", "model")))
    constants = dict(getattr(rg, "constants", {}) or {})
    nodes = _ordered_nodes(rg)
    used = set(rg.inputs) | set(rg.outputs) | set(constants)
    for n in nodes:
        used.update(t for t in list(n.inputs) + list(n.outputs) if t)
    for name, t in rg.tensors.items():
        if name not in used:  # left behind by a fusion: no node reads or writes it
            continue
        dtype = str(_value(t.dtype))
        data = constants.get(name)
        if data is not None:
            data = np.ascontiguousarray(np.asarray(data, dtype=dtype))
            shape = tuple(int(d) for d in data.shape)
        else:
            shape = _dims(t)
        g.add_tensor(TensorInfo(name, shape, dtype, data))
    for name, data in constants.items():  # constants without a tensor entry
        if name not in g.tensors:
            a = np.ascontiguousarray(np.asarray(data))
            g.add_tensor(TensorInfo(name, tuple(a.shape), a.dtype.name, a))
    for n in nodes:
        op = str(_value(n.op_type))
        g.add_node(Node(str(n.name), _OP_ALIASES.get(op, op), list(n.inputs), list(n.outputs),
                        dict(getattr(n, "attrs", {}) or {})))
    g.inputs = list(rg.inputs)
    g.outputs = list(rg.outputs)
    return g


class Mi355xBackend:
    """BackendBase for target "mi355x": generate(ctx) -> CodeGenResult
    (codegen/base.py:32-45). The generated C calls libnnc_hip.so's nnc_*
    entry points on tensors bound into one HBM arena."""

    target = "mi355x"

    def __init__(self, debug_mode: bool = False, repo_root: str | Path | None = None):
        self.debug_mode = debug_mode
        self.repo_root = str(repo_root or REPO_ROOT)
        self.last_program: Program | None = None

    def generate(self, ctx) -> CodeGenResult:
        md = dict(getattr(ctx, "metadata", {}) or {})
        strategy = md.get("memory_strategy")
        if strategy not in (None, "basic", "cost_aware"):
            raise ValueError(f"unknown memory strategy {strategy!r} (basic, cost_aware)")
        max_memory = md.get("max_memory")
        graph = graph_from_context(ctx)
        prog = build_program(graph, int(getattr(ctx, "optimization_level", 0)), strategy,
                             int(max_memory) if max_memory is not None else None)
        debug = bool(self.debug_mode or getattr(ctx, "debug", False))
        result = CodeGenResult()
        for art in codegen.generate(prog, md.get("entry_point", "nnc_run"), self.repo_root, debug_mode=debug):
            result.add_file(art.filename, art.content, art.file_type)
        result.metadata.update({
            "target": self.target,
            "calls": len(prog.calls),
            "arena_bytes": prog.plan.total_bytes,
            "activation_bytes": prog.plan.activation_bytes,
            "spill_bytes": prog.plan.slow_bytes,
        })
        self.last_program = prog
        return result
