"""Which element-wise chains run on a kernel compiled for them (CPU only: the
query is a host-side table lookup in libnnc_hip.so, no HIP call).

nnc_hip_fused_eltwise runs a chain whose steps match an entry of the
library's table on a kernel with those steps as compile-time code, and any
other chain on the general kernel that reads the steps at run time (the GPU
tests check both give the op-by-op bits). Every chain the mi355x O3 compiler
emits for its model set must be in the table."""

from __future__ import annotations

import ctypes

import pytest

from ew_cases import EW_OPS, EW_PROGRAMS, EW_SPECIALIZED


@pytest.fixture(scope="module")
def query(pkg):
    from nnc_py_amd import runtime
    if not runtime.LIB_PATH.exists():
        pytest.fail("libnnc_hip.so is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(runtime.LIB_PATH))
    f = lib.nnc_hip_ew_chain_specialized
    f.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.c_int]
    f.restype = ctypes.c_int

    def ask(n_in, prog):
        arr = (ctypes.c_int * max(len(prog), 1))(*prog)
        return f(n_in, arr, len(prog) // 3)
    return ask


def _prog(steps):
    out = []
    for st in steps:
        out += [EW_OPS[st[0]][0], st[1], st[2]]
    return out


def test_table_membership(query):
    for k, (n_in, steps) in enumerate(EW_PROGRAMS):
        assert query(n_in, _prog(steps)) == (1 if k in EW_SPECIALIZED else 0), k


def test_near_misses_run_on_the_general_kernel(query):
    n_in, steps = EW_PROGRAMS[1]
    prog = _prog(steps)
    assert query(n_in, prog) == 1
    assert query(n_in + 1, prog) == 0  # one more input
    assert query(n_in, prog[:-3]) == 0  # a step fewer
    swapped = list(prog)
    swapped[-1] = 0  # the last add reads input 0, not 2
    assert query(n_in, swapped) == 0
    other_op = list(prog)
    other_op[3 * 3] = EW_OPS["TANH"][0]  # tanh for sigmoid
    assert query(n_in, other_op) == 0
    unary_y = list(prog)
    unary_y[3 * 2 + 2] = 1  # a unary step's y is not compared
    assert query(n_in, unary_y) == 1
    assert query(0, prog) == 0 and query(5, prog) == 0


def test_compiler_chains_are_compiled_kernels(query, pkg):
    """Every nnc_hip_fused_eltwise call of the O3 programs of the model set
    (the bandwidth-chain program has two chains; ResNet-18 and the
    transformer encoder have none) has a kernel compiled for it."""
    from nnc_py_amd.compiler import build_program, zoo
    seen = 0
    for graph in (zoo.bandwidth_chain(seed=1), zoo.resnet18(batch=1, seed=1),
                  zoo.transformer_encoder(batch=8, seq=128)):
        prog = build_program(graph, opt_level=3)
        for call in prog.calls:
            if call.op != "nnc_hip_fused_eltwise":
                continue
            args = dict((i, a) for i, a in enumerate(call.args))
            n_in, steps = args[1][1], args[2][1]
            assert query(n_in, steps) == 1, (call.node, steps)
            seen += 1
    assert seen == 2
