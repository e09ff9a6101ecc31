"""Build and run a lowered program in-process.

build_program() runs the pass pipeline of an optimisation level, plans the
arena and lowers every node to an nnc_* call - the same program the code
generator writes out as model.c/tensors.c. Executor binds it to one
implementation of the ABI and runs nnc_run()'s call sequence through ctypes:

  Executor(prog, device=True)   libnnc_hip.so, one device allocation holding
                                the whole arena (activations + constants)
  Executor(prog, lib=cpu_lib)   a host implementation of the same ABI on a
                                host buffer with the same layout (used by the
                                tests to compare whole networks)
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from .. import abi
from .ir import Graph, Node
from .lower import Call, lower
from .passes import (SPILL_OPS, Branch, MemoryPlan, branch_calls, check_plan, eliminate_dead_code,
                     eliminate_identity, find_branches, fit_memory, fuse_matmul_bias, fuse_patterns, fuse_projection,
                     fuse_residual, pack_conv_weights, plan_memory, prepack_lowering, stream_tiles,
                     eliminate_concat_split, fuse_eltwise_chains, compose_transposes, fuse_add_layernorm,
                     fuse_scaled_softmax, fuse_split_transposes, fuse_attention)


@dataclass
class Program:
    graph: Graph
    order: list[Node]
    plan: MemoryPlan
    calls: list[Call]
    opt_level: int
    branches: list[Branch] = field(default_factory=list)  # side branches on stream 1 (O3)


# Conv -> Add -> Relu fusion into nnc_hip_conv_add_relu at O3 (mi355x target).
RESIDUAL_FUSION = True
# tap-major 3x3 conv weights and nnc_hip_conv_packed at O3 (mi355x target).
PACK_CONV_WEIGHTS = True
# a residual block's 1x1 projection folded into its last 3x3 conv
# (nnc_hip_conv_proj) at O3 (mi355x target).
PROJECTION_FUSION = True
# producer -> consumer tile streaming through a workgroup's on-chip memory
# at O3 (mi355x target): GlobalAveragePool -> Flatten -> Gemm as
# nnc_hip_gap_gemm_nt.
STREAM_TILES = True
# O3: element-wise chains in one pass (nnc_hip_fused_eltwise), Add ->
# LayerNormalization in one pass (nnc_hip_add_layernorm), Div by one element
# -> Softmax in one pass (nnc_hip_scaled_softmax), Concat -> Split round
# trips removed, Transpose -> Transpose composed into one copy, a Split's
# pieces reshaped and transposed straight from the unsplit tensor
ELTWISE_FUSION = True
# independent side branches (ResNet's downsample convolutions) on the second
# library stream at O3 (mi355x target), while the main branch's convolutions
# total at most BRANCH_MAX_FLOPS: two kernels overlap only while neither fills
# the GPU. Off by default: on ResNet-18 the overlap measured 3% slower at
# batch 1 (3261 vs 3374 img/s), +0.4% at batch 8 and -0.4% at batch 32; the
# overlapped 1x1 convolution slows from 10.8 to 14.2 us and the cross-stream
# edges of the captured graph cost more than the overlap saves.
BRANCH_STREAMS = False
# At O3 (mi355x target) a transformer layer's attention block becomes one
# nnc_hip_attention call (passes.fuse_attention).
ATTENTION_FUSION = True
BRANCH_MAX_FLOPS = 1e9


def build_program(graph: Graph, opt_level: int = 1, memory_strategy: str | None = None,
                  max_memory: int | None = None, target_passes: bool = True,
                  branch_streams: bool | None = None) -> Program:
    """Pass pipeline per optimisation level (passes/base.py:67-161 of the
    reference), arena plan, lowering. Mutates `graph`. `target_passes`
    False leaves out the mi355x target's own O3 rewrites (residual fusion,
    MatMul+bias fusion, packed conv weights, view aliasing), giving the call
    sequence of the reference's own O3 pipeline for the reference runtime.
    `branch_streams` (default BRANCH_STREAMS) runs independent side branches
    on the second library stream at O3."""
    if opt_level >= 1:
        eliminate_identity(graph)
        eliminate_dead_code(graph)
    use_branches = opt_level >= 3 and target_passes and (BRANCH_STREAMS if branch_streams is None else branch_streams)
    if opt_level >= 3:
        fuse_patterns(graph)
        if target_passes:
            if RESIDUAL_FUSION:
                fuse_residual(graph)
            fuse_matmul_bias(graph)
            if PACK_CONV_WEIGHTS:
                pack_conv_weights(graph)
                # the downsample conv either joins the residual conv or runs beside it on stream 1
                if PROJECTION_FUSION and RESIDUAL_FUSION and not use_branches:
                    fuse_projection(graph)
        prepack_lowering(graph)
        if target_passes and STREAM_TILES:
            stream_tiles(graph)
        if target_passes and ELTWISE_FUSION:
            eliminate_concat_split(graph)
            compose_transposes(graph)
            fuse_split_transposes(graph)
            fuse_add_layernorm(graph)
            fuse_scaled_softmax(graph)
            if ATTENTION_FUSION:
                fuse_attention(graph)
            fuse_eltwise_chains(graph)
    order = graph.topological_sort()
    branches = find_branches(graph, order, BRANCH_MAX_FLOPS) if use_branches else []
    groups = [[b.side] + b.main for b in branches]
    strategy = memory_strategy or ("basic" if opt_level == 0 else "cost_aware")

    def plan_fn(o, budget=None):
        return plan_memory(graph, o, strategy, None, alias_views=opt_level >= 3 and target_passes,
                           concurrent=groups, budget=budget)

    plan = plan_fn(order, max_memory)
    if max_memory is not None and plan.activation_bytes > max_memory:
        if strategy != "cost_aware":
            raise ValueError(f"max_memory ({max_memory}) < peak activation footprint ({plan.activation_bytes}) "
                             f"of the {strategy} plan; spilling needs the cost_aware strategy")
        branches, groups = [], []  # spills go between the nodes of one stream
        order, plan = fit_memory(graph, order, max_memory, plan_fn)
    check_plan(graph, order, plan, groups)
    calls = branch_calls(lower(graph, order, plan.aliases), branches, lambda op, args: Call(op, args, ""))
    return Program(graph, order, plan, calls, opt_level, branches)


class Executor:
    def __init__(self, prog: Program, device: bool = True, lib: ctypes.CDLL | None = None):
        self.prog = prog
        self.device = device
        g, plan = prog.graph, prog.plan
        if device:
            from .. import runtime
            self.rt = runtime
            self.lib = lib or runtime.load()
            self.base = self.lib.nnc_hip_malloc(plan.total_bytes)
            if not self.base:
                raise runtime.HipError(f"cannot allocate a {plan.total_bytes}-byte arena")
        else:
            if lib is None:
                raise ValueError("a host executor needs an ABI library")
            self.lib = lib
            self._host = np.zeros(plan.total_bytes + 256, np.uint8)
            addr = self._host.ctypes.data
            self.base = addr + (-addr % 256)
        self._keep = []
        self.slow = None  # spill pool: pinned host memory on a device, host memory otherwise
        if plan.slow_bytes:
            if device:
                self.slow = self.lib.nnc_hip_host_malloc(plan.slow_bytes)
                if not self.slow:
                    raise runtime.HipError(f"cannot allocate a {plan.slow_bytes}-byte spill pool")
            else:
                self._slow_host = np.zeros(plan.slow_bytes + 256, np.uint8)
                addr = self._slow_host.ctypes.data
                self.slow = addr + (-addr % 256)
        self.tensors: dict[str, abi.Tensor] = {}
        places = [(n, self.base + off) for n, off in plan.offsets.items()]
        places += [(n, self.slow + off) for n, off in plan.slow_offsets.items()]
        for name, addr in places:
            t = g.tensors[name]
            ten, sh = abi.make_tensor(addr, abi.NUMPY_TO_NNC[t.dtype], t.shape, t.nbytes)
            self._keep.append(sh)
            self.tensors[name] = ten
        for name, t in g.constants.items():
            self._write(name, t.data)
        self._calls = [(self._fn(c.op), self._args(c)) for c in prog.calls]

    # -- memory --------------------------------------------------------------
    def _addr(self, name: str) -> int:
        return self.base + self.prog.plan.offsets[name]

    def _write(self, name: str, arr: np.ndarray) -> None:
        t = self.prog.graph.tensors[name]
        a = np.ascontiguousarray(arr, dtype=t.dtype)
        assert a.nbytes == t.nbytes, (name, a.shape, t.shape)
        if self.device:
            self.rt.check(self.lib.nnc_hip_memcpy_h2d(self._addr(name), a.ctypes.data, a.nbytes), "upload")
        else:
            ctypes.memmove(self._addr(name), a.ctypes.data, a.nbytes)

    def _read(self, name: str) -> np.ndarray:
        t = self.prog.graph.tensors[name]
        out = np.empty(t.shape, t.dtype)
        if self.device:
            self.rt.check(self.lib.nnc_hip_memcpy_d2h(out.ctypes.data, self._addr(name), t.nbytes), "download")
        else:
            ctypes.memmove(out.ctypes.data, self._addr(name), t.nbytes)
        return out

    def set_input(self, name: str, arr: np.ndarray) -> None:
        self._write(name, arr)

    def get(self, name: str) -> np.ndarray:
        if self.device:
            self.rt.sync()
        return self._read(name)

    # -- calls ---------------------------------------------------------------
    def _fn(self, op: str):
        """The library's entry point; the stream fork/select/join calls are
        no-ops on an implementation without them (a host library runs every
        call in order anyway)."""
        if op.startswith("nnc_hip_stream_") and not hasattr(self.lib, op):
            return lambda *args: 0
        return getattr(self.lib, op)

    def _args(self, call: Call) -> tuple:
        out = []
        for spec in call.args:
            kind = spec[0]
            if kind == "t":
                out.append(ctypes.pointer(self.tensors[spec[1]]))
            elif kind == "tv":
                t = self.prog.graph.tensors[spec[1]]
                ten, sh = abi.make_tensor(self._addr(spec[1]), abi.NUMPY_TO_NNC[t.dtype], spec[2], t.nbytes)
                self._keep += [ten, sh]
                out.append(ctypes.pointer(ten))
            elif kind == "null" or kind == "i64null":
                out.append(None)
            elif kind == "i":
                out.append(int(spec[1]))
            elif kind == "f":
                out.append(float(spec[1]))
            elif kind == "tl":
                arr = (abi.TP * len(spec[1]))(*[ctypes.pointer(self.tensors[n]) for n in spec[1]])
                self._keep.append(arr)
                out.append(ctypes.cast(arr, abi.TPP))
            elif kind == "i64":
                arr = (ctypes.c_int64 * max(1, len(spec[1])))(*[int(v) for v in spec[1]])
                self._keep.append(arr)
                out.append(ctypes.cast(arr, abi.I64P))
            elif kind == "i32":
                arr = (ctypes.c_int * max(1, len(spec[1])))(*[int(v) for v in spec[1]])
                self._keep.append(arr)
                out.append(ctypes.cast(arr, abi.I32P))
            elif kind == "f32":
                arr = (ctypes.c_float * max(1, len(spec[1])))(*[float(v) for v in spec[1]])
                self._keep.append(arr)
                out.append(ctypes.cast(arr, abi.F32P))
            else:
                raise ValueError(f"unknown argument kind {kind!r}")
        return tuple(out)

    def run(self) -> None:
        """One nnc_run(): every call in order (asynchronous on the device)."""
        for fn, args in self._calls:
            fn(*args)

    def run_debug(self, path) -> None:
        """One nnc_run() node by node, writing every node's outputs after it
        runs to `path` in the debug dump format (nnc_py_amd.tools.
        debug_compare): the counterpart of the generated program's debug
        mode. Node indices count the non-constant nodes in topological order,
        as the reference's dump injection (model_source.py:398-428)."""
        from ..tools.debug_compare import write_tensor
        by_node: dict[str, list] = {}
        for call, fn_args in zip(self.prog.calls, self._calls):
            by_node.setdefault(call.node, []).append(fn_args)
        consts = self.prog.graph.constants
        with open(path, "w") as f:
            idx = 0
            for node in self.prog.order:
                for fn, args in by_node.get(node.name, []):
                    fn(*args)
                if node.op_type in SPILL_OPS:  # the compiler's copies, not graph nodes
                    continue
                for out in node.outputs:
                    if out in consts or out not in self.prog.plan.offsets:
                        continue
                    write_tensor(f, out, idx, self.get(out))
                idx += 1

    def capture(self) -> None:
        """Record run() into a hipGraph (device only); replay() launches it."""
        self.rt.check(self.lib.nnc_hip_graph_begin(), "nnc_hip_graph_begin")
        try:
            self.run()
        finally:
            self.rt.check(self.lib.nnc_hip_graph_end(), "nnc_hip_graph_end")

    def replay(self) -> None:
        self.rt.check(self.lib.nnc_hip_graph_launch(), "nnc_hip_graph_launch")

    def close(self) -> None:
        if self.device and self.base:
            self.lib.nnc_hip_free(self.base)
            self.base = None
        if self.device and self.slow:
            self.lib.nnc_hip_host_free(self.slow)
            self.slow = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
