"""A fast-memory budget below the plan's peak: spill and reload.

The reference meets `max_memory` by spilling tensors from its fast pool to a
slow pool and copying them back before their next use
(passes/strategies/cost_aware_allocator.py:63-377, spill copies in
codegen/x86_emitters/model_source.py:259-290); its tests check that the fast
pool stays within the limit (tests/test_compaction.py:597-640,
tests/test_overflow_e2e.py:77-345), that a budget below one node's demand is
rejected (tests/test_compaction.py:98-110) and that spilled programs compute
what unspilled ones do (tests/test_spill_correctness.py:464-632). Here the
arena's activation region is the fast pool and pinned host memory the slow
one; a spill or reload is one byte copy, so a budgeted program's outputs must
equal the unbudgeted program's bit for bit.
"""

from __future__ import annotations

import subprocess

import numpy as np
import pytest

import caserun


def _chain():
    """x -> a -> b -> c (softmax: no in-place reuse), out = a + c: a is read
    again after two nodes, so a 4-buffer peak (x, a, b, c at node c) meets a
    3-buffer budget only by spilling a."""
    from nnc_py_amd.compiler import GraphBuilder
    b = GraphBuilder("chain")
    x = b.input("x", (8, 8))
    a = b.softmax(x, name="sa", out="a")
    bb = b.softmax(a, name="sb", out="b")
    c = b.softmax(bb, name="sc", out="c")
    b.output(b.add(a, c, name="add", out="out"))
    return b.build()


def _run_host(prog, oracle_lib, x, name="x"):
    from nnc_py_amd.compiler import Executor
    ex = Executor(prog, device=False, lib=oracle_lib)
    ex.set_input(name, x)
    ex.run()
    out = ex.get(prog.graph.outputs[0])
    ex.close()
    return out


def test_chain_spills_the_long_lived_tensor(pkg, oracle_lib):
    from nnc_py_amd.compiler import build_program
    from nnc_py_amd.compiler.passes import check_plan
    free = build_program(_chain(), opt_level=1)
    assert free.plan.activation_bytes == 4 * 256 and not free.plan.slow_offsets
    prog = build_program(_chain(), opt_level=1, max_memory=3 * 256)
    assert prog.plan.activation_bytes <= 3 * 256
    check_plan(prog.graph, prog.order, prog.plan)
    ops = [(n.op_type, n.inputs[0]) for n in prog.order]
    assert ops == [("Softmax", "x"), ("Softmax", "a"), ("Spill", "a"), ("Softmax", "b"),
                   ("Reload", "a.spilled"), ("Add", "a.reloaded")]
    assert [c.op for c in prog.calls].count("nnc_hip_transfer") == 2
    assert prog.plan.slow_offsets == {"a.spilled": 0} and prog.plan.slow_bytes == 256
    x = np.random.default_rng(0).standard_normal((8, 8)).astype(np.float32)
    assert caserun.same_bits(_run_host(prog, oracle_lib, x), _run_host(free, oracle_lib, x))


def test_budget_below_one_nodes_demand_is_rejected(pkg):
    from nnc_py_amd.compiler import build_program, zoo
    with pytest.raises(ValueError, match="max_memory"):
        build_program(_chain(), opt_level=1, max_memory=2 * 256)
    with pytest.raises(ValueError, match="max_memory"):  # the input alone is larger
        build_program(zoo.resnet18(batch=4, seed=0), opt_level=1, max_memory=1 << 20)
    with pytest.raises(ValueError, match="cost_aware"):  # basic never reuses, so spills free nothing
        build_program(_chain(), opt_level=0, max_memory=3 * 256)
    assert build_program(_chain(), opt_level=0, max_memory=3 * 256, memory_strategy="cost_aware").plan.slow_bytes


def _hourglass(rows=8, cols=64):
    """Encoder a1..a4 (softmax), decoder b3 = a4 + a3, b2 = b3 + a2,
    out = b2 + a1: five buffers live at a4 without a budget, three with
    a1 and a2 spilled until the decoder reads them."""
    from nnc_py_amd.compiler import GraphBuilder
    b = GraphBuilder("hourglass")
    x = b.input("x", (rows, cols))
    a1 = b.softmax(x, name="e1", out="a1")
    a2 = b.softmax(a1, name="e2", out="a2")
    a3 = b.softmax(a2, name="e3", out="a3")
    a4 = b.softmax(a3, name="e4", out="a4")
    b3 = b.add(a4, a3, name="d3", out="b3")
    b2 = b.add(b3, a2, name="d2", out="b2")
    b.output(b.add(b2, a1, name="d1", out="out"))
    return b.build()


def test_hourglass_spills_both_skips(pkg, oracle_lib):
    from nnc_py_amd.compiler import build_program
    from nnc_py_amd.compiler.passes import check_plan
    buf = 8 * 64 * 4
    free = build_program(_hourglass(), opt_level=1)
    assert free.plan.activation_bytes == 5 * buf
    prog = build_program(_hourglass(), opt_level=1, max_memory=3 * buf)
    assert prog.plan.activation_bytes <= 3 * buf
    check_plan(prog.graph, prog.order, prog.plan)
    assert sorted(n.inputs[0] for n in prog.order if n.op_type == "Spill") == ["a1", "a2"]
    x = np.random.default_rng(1).standard_normal((8, 64)).astype(np.float32)
    assert caserun.same_bits(_run_host(prog, oracle_lib, x), _run_host(free, oracle_lib, x))


@pytest.mark.parametrize("opt", [1, 3])
def test_transformer_under_a_budget_matches_the_free_plan(pkg, oracle_lib, opt, monkeypatch):
    """The transformer encoder's residual stream is live across attention and
    the FFN: under a budget below its free peak it is spilled. The fast
    region stays within the budget, every reload precedes the reads of the
    tensor it restores, nothing reads the spilled name after its reload, the
    plan passes its invariants, and the program computes the unbudgeted
    program's bytes on the oracle. (ResNet-18 and LeNet-5 reach their free
    peak inside one node - the stem convolution with the image, the first
    convolution - so no budget below it is feasible for them. With the
    residual Add fused into its LayerNorm the encoder's O3 peak is the FFN
    MatMul's own input and output, 20% below the unfused peak and likewise
    unspillable, so the budgets run on the unfused program.)"""
    from nnc_py_amd.compiler import build_program, executor, zoo
    from nnc_py_amd.compiler.passes import check_plan

    monkeypatch.setattr(executor, "ELTWISE_FUSION", False)

    def graph():
        return zoo.transformer_encoder(batch=2, seq=64)

    free = build_program(graph(), opt_level=opt)
    budget = int(free.plan.activation_bytes * 0.9)
    prog = build_program(graph(), opt_level=opt, max_memory=budget)
    assert prog.plan.activation_bytes <= budget < free.plan.activation_bytes
    check_plan(prog.graph, prog.order, prog.plan)
    assert any(n.op_type == "Spill" for n in prog.order) and prog.plan.slow_bytes > 0
    pos = {n.name: i for i, n in enumerate(prog.order)}
    for k, n in enumerate(prog.order):
        if n.op_type == "Reload":
            back, held = n.outputs[0], n.inputs[0]
            src = next(m for m in prog.order if m.outputs == [held])
            assert src.op_type == "Spill" and pos[src.name] < k
            assert all(pos[m.name] > k for m in prog.order if back in m.inputs)
            assert not any(src.inputs[0] in m.inputs for m in prog.order[k:])
    name = free.graph.inputs[0]
    x = np.random.default_rng(3).standard_normal(free.graph.tensors[name].shape).astype(np.float32)
    assert caserun.same_bits(_run_host(prog, oracle_lib, x, name), _run_host(free, oracle_lib, x, name))


def test_generated_c_with_a_spill_pool_runs_on_the_oracle(tmp_path, pkg, oracle_lib):
    """tensors.c reserves and binds the spill pool; model.c copies through
    nnc_hip_transfer; the host build computes what the executor does."""
    from nnc_py_amd.compiler import build_program
    from nnc_py_amd.compiler.compiler import Compiler
    from test_codegen import _build_with_shim, _parse_outputs
    budget = 3 * 8 * 64 * 4
    Compiler(target="mi355x", opt_level=1).compile(_hourglass(), str(tmp_path), max_memory=str(budget))
    tensors_c = (tmp_path / "tensors.c").read_text()
    assert "nnc_hip_spill_reserve(NNC_SPILL_SIZE)" in tensors_c
    act = int(next(l.split()[2] for l in tensors_c.splitlines() if l.startswith("#define NNC_ACTIVATION_BYTES")))
    assert act <= budget
    assert (tmp_path / "model.c").read_text().count("nnc_hip_transfer(") == 4
    exe = _build_with_shim(tmp_path)
    run = subprocess.run([str(exe), str(tmp_path / "constants.bin"), "1"], capture_output=True, text=True,
                         timeout=60)
    assert run.returncode == 0, run.stderr
    x = (np.arange(8 * 64, dtype=np.float32) * np.float32(0.01)).reshape(8, 64)
    want = _run_host(build_program(_hourglass(), opt_level=1), oracle_lib, x)
    np.testing.assert_allclose(_parse_outputs(run.stdout), want.ravel()[:10], rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [2, 8])
def test_transformer_under_a_budget_on_the_gpu(hip, batch, monkeypatch):
    """HBM arena as the fast pool, pinned host memory as the spill pool:
    eager and three graph replays equal the unbudgeted GPU program bit for
    bit (the same kernels; spills and reloads are exact copies). The
    unfused program: the fused one peaks inside one node."""
    from nnc_py_amd import runtime
    from nnc_py_amd.compiler import Executor, build_program, executor, zoo

    monkeypatch.setattr(executor, "ELTWISE_FUSION", False)

    def graph():
        return zoo.transformer_encoder(batch=batch, seq=128)

    free_prog = build_program(graph(), opt_level=3)
    name = free_prog.graph.inputs[0]
    x = np.random.default_rng(7).standard_normal(free_prog.graph.tensors[name].shape).astype(np.float32)
    free = Executor(free_prog, device=True)
    free.set_input(name, x)
    free.run()
    want = free.get(free_prog.graph.outputs[0])
    budget = int(free_prog.plan.activation_bytes * 0.9)
    free.close()
    prog = build_program(graph(), opt_level=3, max_memory=budget)
    n_spills = sum(n.op_type == "Spill" for n in prog.order)
    print(f"transformer b{batch}: budget {budget}, {n_spills} spills, {prog.plan.slow_bytes} B pool", flush=True)
    assert n_spills
    ex = Executor(prog, device=True)
    ex.set_input(name, x)
    ex.run()
    assert caserun.same_bits(ex.get(prog.graph.outputs[0]), want)
    ex.capture()
    for _ in range(3):
        ex.replay()
        runtime.sync()
        assert caserun.same_bits(ex.get(prog.graph.outputs[0]), want)
        ex.run()
        runtime.sync()
    ex.close()


@pytest.mark.gpu
def test_generated_model_with_a_spill_pool_on_the_gpu(tmp_path, hip, oracle_lib):
    """The generated program with a spill pool, built with make against
    libnnc_hip.so: first call eager, second captured, third replayed."""
    from nnc_py_amd.compiler import build_program
    from nnc_py_amd.compiler.compiler import Compiler
    from test_codegen import _parse_outputs
    budget = 3 * 8 * 64 * 4
    Compiler(target="mi355x", opt_level=1).compile(_hourglass(), str(tmp_path), max_memory=str(budget))
    assert "NNC_SPILL_SIZE" in (tmp_path / "tensors.c").read_text()
    subprocess.run(["make", "-C", str(tmp_path), "-j4"], check=True, capture_output=True, text=True)
    print("built the generated hourglass model with a spill pool", flush=True)
    run = subprocess.run([str(tmp_path / "model"), str(tmp_path / "constants.bin"), "3"], capture_output=True,
                         text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    got = _parse_outputs(run.stdout)
    x = (np.arange(8 * 64, dtype=np.float32) * np.float32(0.01)).reshape(8, 64)
    want = _run_host(build_program(_hourglass(), opt_level=1), oracle_lib, x).ravel()[:10]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
