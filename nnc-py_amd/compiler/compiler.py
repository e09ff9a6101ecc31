"""Compiler(target="mi355x", opt_level=...).compile(...) - the reference API
(src/nnc_py/compiler.py:103-264) with the MI355X target.

    from nnc_py_amd.compiler.compiler import Compiler
    Compiler(target="mi355x", opt_level=3).compile(graph_or_onnx, "out/",
                                                   entry_point="nnc_run")

writes model.c / model.h / tensors.c / constants.bin / constants_loader.c /
test_runner.c / Makefile into output_dir; `make` builds ./model and
libmodel.so against libnnc_hip.so.
"""

from __future__ import annotations

import re
from collections.abc import Mapping
from pathlib import Path
from typing import Any

from .backend import CodeGenResult, CompileContext, Mi355xBackend
from .executor import Program
from .ir import Graph

REPO_ROOT = Path(__file__).resolve().parents[2]

_SIZE = re.compile(r"^(\d+(?:\.\d+)?)\s*([KMGT]?)B?$")
_UNIT = {"": 1, "K": 1 << 10, "M": 1 << 20, "G": 1 << 30, "T": 1 << 40}


def parse_memory_size(size_str: str | None) -> int | None:
    """'256K' -> 262144, '16MB' -> 16777216, '512' -> 512 (compiler.py:19-64)."""
    if size_str is None:
        return None
    m = _SIZE.match(str(size_str).strip().upper())
    if not m:
        raise ValueError(f"Invalid memory size format: {size_str}")
    return int(float(m.group(1)) * _UNIT[m.group(2)])


TARGETS = ("mi355x",)


class Compiler:
    """Graph (or ONNX file) -> C code calling libnnc_hip through the nnc ABI."""

    def __init__(self, target: str = "mi355x", opt_level: int = 0, memory_strategy: str | None = None,
                 enable_constant_folding: bool = True, debug_mode: bool = False,
                 cost_model_cli_command: str | list[str] | None = None,
                 metadata: Mapping[str, Any] | None = None):
        self.target = target
        self.opt_level = int(opt_level)
        self.memory_strategy = memory_strategy
        self.enable_constant_folding = enable_constant_folding
        self.debug_mode = debug_mode
        self.cost_model_cli_command = cost_model_cli_command
        self.default_metadata = dict(metadata or {})
        self._check_target(target)
        self.last_program: Program | None = None
        self.last_artifacts: CodeGenResult | None = None

    @staticmethod
    def _check_target(target: str) -> None:
        if target == "mi355x":
            return
        if target == "npu":  # the reference's placeholder target (compiler.py:278-282)
            raise NotImplementedError("NPU backend is not implemented yet. Use target='mi355x'.")
        if target == "x86":
            raise ValueError("target 'x86' is the reference nnc-py backend; this package provides 'mi355x'")
        raise ValueError(f"Unknown target: {target}")

    def _create_backend(self, target: str) -> Mi355xBackend:
        """The backend for `target` (compiler.py:266-285 of the reference,
        whose _create_backend gains the same "mi355x" branch)."""
        self._check_target(target)
        return Mi355xBackend(debug_mode=self.debug_mode, repo_root=REPO_ROOT)

    def _load(self, model) -> Graph:
        if isinstance(model, Graph):
            return model
        path = Path(model)
        if path.suffix == ".onnx":
            from .onnx_reader import load_onnx
            return load_onnx(path)
        raise ValueError(f"cannot compile {model!r}: expected a Graph or an .onnx file")

    def compile(self, model, output_dir: str, entry_point: str = "nnc_run", max_memory: str | None = None,
                memory_strategy: str | None = None, cost_model_cli_command=None,
                metadata: Mapping[str, Any] | None = None) -> Program:
        """Same stages as the reference's compile (compiler.py:128-264): load,
        a CompileContext with entry_point / max_memory / memory_strategy in its
        metadata, then the backend's generate(ctx) - here Mi355xBackend, which
        also runs this target's passes - and the files written out."""
        graph = self._load(model)
        strategy = memory_strategy or self.memory_strategy
        md = dict(self.default_metadata)
        md.update(dict(metadata or {}))
        if cost_model_cli_command is not None:
            md["cost_model_cli_command"] = cost_model_cli_command
        md["entry_point"] = entry_point
        if max_memory is not None:
            md["max_memory"] = parse_memory_size(max_memory)
        if strategy is not None:
            md["memory_strategy"] = strategy
        ctx = CompileContext(graph, self.target, self.opt_level, self.debug_mode, md)
        backend = self._create_backend(self.target)
        artifacts = backend.generate(ctx)
        out = Path(output_dir)
        out.mkdir(parents=True, exist_ok=True)
        for art in artifacts.files:
            path = out / art.filename
            if art.file_type == "binary":
                path.write_bytes(art.content)
            else:
                path.write_text(art.content)
        artifacts.metadata.update({"entry_point": entry_point, "target": self.target, "opt_level": self.opt_level})
        self.last_artifacts = artifacts
        self.last_program = backend.last_program
        return backend.last_program
