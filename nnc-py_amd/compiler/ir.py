"""Graph IR consumed by the MI355X target.

Mirrors the reference IR's content (src/nnc_py/ir/graph.py:12-88,
ir/node.py:8-124, ir/tensor.py:10-53): named tensors with static shapes and a
dtype, nodes carrying an ONNX op type string, attribute dict and free-form
metadata (lowering decisions such as the conv kernel kind,
passes/prepack_lowering.py:48-79). Op type strings are the reference's
OpType values ("Conv", "Relu", "FusedConvRelu", ...).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import numpy as np

# dtype name -> bytes per element
DTYPE_SIZE = {"float32": 4, "float16": 2, "int64": 8, "int32": 4, "int8": 1, "uint8": 1, "bool": 1}

# op types (reference ir/node.py:8-92)
FUSED = {
    "FusedConvRelu": ("Conv", "Relu"),
    "FusedConvSigmoid": ("Conv", "Sigmoid"),
    "FusedAddRelu": ("Add", "Relu"),
    "FusedAddSigmoid": ("Add", "Sigmoid"),
    "FusedMatMulRelu": ("MatMul", "Relu"),
    "FusedConvAddRelu": ("Conv", "Add", "Relu"),
    "FusedMatMulBias": ("MatMul", "Add"),
    "FusedMatMulBiasRelu": ("MatMul", "Add", "Relu"),
}


@dataclass
class TensorInfo:
    name: str
    shape: tuple
    dtype: str = "float32"
    data: np.ndarray | None = None  # constants only
    pool: str = "fast"  # "slow": a spilled copy in the spill pool (pinned host memory)

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= int(s)
        return n

    @property
    def nbytes(self) -> int:
        return self.numel * DTYPE_SIZE[self.dtype]

    @property
    def is_constant(self) -> bool:
        return self.data is not None


@dataclass
class Node:
    name: str
    op_type: str
    inputs: list[str]
    outputs: list[str]
    attrs: dict[str, Any] = field(default_factory=dict)
    metadata: dict[str, Any] = field(default_factory=dict)


class Graph:
    """Tensors by name, nodes in a valid topological order."""

    def __init__(self, name: str = "model"):
        self.name = name
        self.tensors: dict[str, TensorInfo] = {}
        self.nodes: list[Node] = []
        self.inputs: list[str] = []
        self.outputs: list[str] = []

    # -- construction ------------------------------------------------------
    def add_tensor(self, t: TensorInfo) -> TensorInfo:
        if t.name in self.tensors:
            raise ValueError(f"duplicate tensor {t.name!r}")
        self.tensors[t.name] = t
        return t

    def add_node(self, node: Node) -> Node:
        self.nodes.append(node)
        return node

    @property
    def constants(self) -> dict[str, TensorInfo]:
        return {n: t for n, t in self.tensors.items() if t.is_constant}

    def consumers(self, tensor: str) -> list[Node]:
        return [n for n in self.nodes if tensor in n.inputs]

    def producer(self, tensor: str) -> Node | None:
        for n in self.nodes:
            if tensor in n.outputs:
                return n
        return None

    def topological_sort(self) -> list[Node]:
        """Nodes ordered so every input is produced before use; stable with
        respect to insertion order (the reference sorts with networkx,
        graph.py:55-60; insertion order is already topological here unless a
        pass appended nodes out of order)."""
        ready = set(self.inputs) | set(self.constants)
        order, pending = [], list(self.nodes)
        while pending:
            progressed = False
            rest = []
            for n in pending:
                if all(i in ready or i == "" for i in n.inputs):
                    order.append(n)
                    ready.update(n.outputs)
                    progressed = True
                else:
                    rest.append(n)
            if not progressed:
                raise ValueError(f"graph has a cycle or a missing producer: {[n.name for n in rest]}")
            pending = rest
        return order
