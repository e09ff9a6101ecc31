"""nnc compiler pipeline for the mi355x target: graph IR, passes, arena plan,
lowering to nnc_* calls, C code generation and an in-process executor."""

from .builder import GraphBuilder  # noqa: F401
from .executor import Executor, Program, build_program  # noqa: F401
from .ir import Graph, Node, TensorInfo  # noqa: F401
