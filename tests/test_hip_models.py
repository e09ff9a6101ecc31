"""Whole-network parity of the HIP path against the oracle.

1. Per op on identical inputs: the oracle runs ResNet-18 (and LeNet-5) with a
   no-reuse arena so every intermediate survives; each nnc_* call of the
   program is then replayed alone on the GPU from the oracle's inputs and
   compared with the oracle's output of that call, at the ResNet-18 layer
   shapes (batch 1, 2 and the benchmark's batch 32, whose kernel choices -
   tile shapes, stream-K splits, in-kernel finishes and fixups - differ from
   the smaller batches'). Bar: 1e-4 abs / 1e-3 rel, bit-exact for pools and
   copies.
2. End to end: logits of the GPU program vs the oracle program. Errors
   compound over 20 unnormalised layers, so the bar is the reference's own
   ResNet end-to-end bar (rtol 1.5e-2, atol 3e-3; tests/test_common.py:545).
3. Size-independent property at batch 32: every image's logits equal the
   batch-1 logits of that image (tiles and K splits differ between the two).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import caserun

pytestmark = pytest.mark.gpu

EXACT_OPS = {"nnc_maxpool2d", "nnc_avgpool2d", "nnc_flatten", "nnc_reshape", "nnc_relu", "nnc_add",
             "nnc_add_relu", "nnc_transpose", "nnc_concat", "nnc_split", "nnc_identity"}


def _programs(build, graph_fn, opt_level):
    from nnc_py_amd.compiler import build_program
    return build_program(graph_fn(), opt_level=opt_level, memory_strategy="basic")


def _oracle_trace(prog, oracle_lib, x):
    from nnc_py_amd.compiler import Executor
    ex = Executor(prog, device=False, lib=oracle_lib)
    ex.set_input("input", x)
    ex.run()
    return {name: ex.get(name) for name in prog.plan.offsets}


def _call_case(prog, call, values):
    """A caserun case replaying one call of the program on stored tensors."""
    g = prog.graph
    tensors, args = {}, []
    for spec in call.args:
        if spec[0] == "t":
            tensors[spec[1]] = values[spec[1]]
            args.append(spec)
        elif spec[0] == "tv":
            key = spec[1] + "::view"
            tensors[key] = values[spec[1]].reshape(spec[2])
            args.append(("t", key))
        elif spec[0] == "tl":
            for n in spec[1]:
                tensors[n] = values[n]
            args.append(spec)
        else:
            args.append(spec)
    node = next(n for n in prog.order if n.name == call.node)
    outs = [o for o in node.outputs]
    for o in outs:
        tensors[o] = np.zeros(g.tensors[o].shape, g.tensors[o].dtype)
    return {"name": call.node, "op": call.op, "tensors": tensors, "args": args, "outputs": outs}


@pytest.mark.parametrize("model,batch,opt", [("resnet18", 1, 3), ("resnet18", 2, 1), ("resnet18", 32, 3),
                                             ("lenet5", 1, 1), ("lenet5", 3, 3)])
def test_per_op_parity_on_oracle_activations(model, batch, opt, hip, dmem, abi, oracle_lib):
    from nnc_py_amd.compiler import zoo
    fn = {"resnet18": lambda: zoo.resnet18(batch=batch, seed=1),
          "lenet5": lambda: zoo.lenet5(batch=batch, seed=1)}[model]
    prog = _programs(None, fn, opt)
    shape = prog.graph.tensors["input"].shape
    x = np.random.default_rng(0).standard_normal(shape).astype(np.float32)
    values = _oracle_trace(prog, oracle_lib, x)
    failures = []
    for call in prog.calls:
        if not call.node:  # stream fork/select/join: no tensors
            continue
        case = _call_case(prog, call, values)
        print(f"{model} b{batch} O{opt}: {call.op} {call.node}", flush=True)
        got = caserun.run_case(hip, case, abi, dmem)
        for key in case["outputs"]:
            want = values[key]
            if call.op in EXACT_OPS:
                if not caserun.same_bits(got[key], want):
                    failures.append(f"{call.node} ({call.op}): not bit-exact")
            else:
                bad = caserun.fp_violations(got[key], want, 1e-4, 1e-3)
                if bad.size:
                    d = np.abs(got[key].ravel()[bad] - want.ravel()[bad])
                    failures.append(f"{call.node} ({call.op}): {bad.size}/{want.size} outside bar, "
                                    f"max diff {d.max():.3g}")
        dmem.release()
    assert not failures, "\n".join(failures)


def _e2e(graph_fn, x, hip_opt, oracle_lib):
    from nnc_py_amd.compiler import Executor, build_program
    dev = Executor(build_program(graph_fn(), opt_level=hip_opt), device=True)
    dev.set_input("input", x)
    dev.run()
    got = dev.get("output")
    dev.close()
    host = Executor(build_program(graph_fn(), opt_level=1), device=False, lib=oracle_lib)
    host.set_input("input", x)
    host.run()
    return got, host.get("output")


def test_resnet18_end_to_end_b1(hip, oracle_lib):
    from nnc_py_amd.compiler import zoo
    x = np.random.default_rng(0).standard_normal((1, 3, 224, 224)).astype(np.float32)
    got, want = _e2e(lambda: zoo.resnet18(batch=1, seed=1), x, 3, oracle_lib)
    bad = caserun.fp_violations(got, want, 3e-3, 1.5e-2)
    rel = np.abs(got - want).max() / np.abs(want).max()
    print(f"resnet18 b1 logits: max |diff| {np.abs(got - want).max():.3g}, relative to max |logit| {rel:.3g}")
    assert bad.size == 0, f"{bad.size} logits outside rtol 1.5e-2 / atol 3e-3"
    assert np.argmax(got) == np.argmax(want)


def test_lenet5_end_to_end(hip, oracle_lib):
    from nnc_py_amd.compiler import zoo
    x = np.random.default_rng(2).standard_normal((4, 1, 28, 28)).astype(np.float32)
    got, want = _e2e(lambda: zoo.lenet5(batch=4, seed=1), x, 3, oracle_lib)
    assert caserun.fp_violations(got, want, 1e-4, 1e-3).size == 0


def test_resnet18_benchmark_program_b32_end_to_end(hip, oracle_lib):
    """The program bench.py times - ResNet-18 at batch 32, O3 with this
    target's passes and the default cost_aware plan (residual convolutions
    written in place over their skip tensors, the stem's max pool inside
    its row kernel, folded projections, 128x128 stream-K tiles with fixups)
    - against the oracle running ResNet-18 at O1 on the same input: every
    logit of all 32 images within the reference's end-to-end ResNet bar
    (rtol 1.5e-2, atol 3e-3), the same top-1 class per image; then captured
    and replayed as a hipGraph three times, each replay bit-identical to
    the eager run."""
    from nnc_py_amd import runtime
    from nnc_py_amd.compiler import Executor, build_program, zoo
    x = np.random.default_rng(0).standard_normal((32, 3, 224, 224)).astype(np.float32)
    prog = build_program(zoo.resnet18(batch=32, seed=1), opt_level=3)
    ops = {c.op for c in prog.calls}
    assert {"nnc_hip_conv_packed", "nnc_hip_conv_proj", "nnc_hip_conv_maxpool"} <= ops, ops
    print("resnet18 b32 O3 benchmark program: eager run", flush=True)
    dev = Executor(prog, device=True)
    dev.set_input("input", x)
    dev.run()
    got = dev.get("output")
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    dev.capture()
    for rep in range(3):
        print(f"resnet18 b32 O3 benchmark program: graph replay {rep}", flush=True)
        dev.replay()
        runtime.sync()
        assert caserun.same_bits(dev.get("output"), got), f"replay {rep} differs from the eager run"
    dev.close()
    print("resnet18 b32: oracle program (O1)", flush=True)
    host = Executor(build_program(zoo.resnet18(batch=32, seed=1), opt_level=1), device=False, lib=oracle_lib)
    host.set_input("input", x)
    host.run()
    want = host.get("output")
    bad = caserun.fp_violations(got, want, 3e-3, 1.5e-2)
    print(f"resnet18 b32 logits: max |diff| {np.abs(got - want).max():.3g}", flush=True)
    assert bad.size == 0, f"{bad.size} of {want.size} logits outside rtol 1.5e-2 / atol 3e-3"
    assert (np.argmax(got, axis=1) == np.argmax(want, axis=1)).all()


def test_resnet18_batch32_matches_batch1_per_image(hip):
    from nnc_py_amd.compiler import Executor, build_program, zoo
    x = np.random.default_rng(0).standard_normal((32, 3, 224, 224)).astype(np.float32)
    big = Executor(build_program(zoo.resnet18(batch=32, seed=1), opt_level=3), device=True)
    big.set_input("input", x)
    big.run()
    y32 = big.get("output")
    big.close()
    one = Executor(build_program(zoo.resnet18(batch=1, seed=1), opt_level=3), device=True)
    for i in (0, 13, 31):
        one.set_input("input", x[i:i + 1])
        one.run()
        y1 = one.get("output")
        bad = caserun.fp_violations(y32[i:i + 1], y1, 3e-3, 1.5e-2)
        assert bad.size == 0, f"image {i}: {bad.size} logits differ between batch 32 and batch 1"
    one.close()


@pytest.mark.parametrize("batch", [1, 8])
def test_branch_streams_match_one_stream(hip, batch):
    """Downsample branches on the second stream (fork/select/join): the
    eager run and three graph replays give the one-stream result bit for bit
    (the same kernels, each on its own per-stream scratch)."""
    from nnc_py_amd import runtime
    from nnc_py_amd.compiler import Executor, build_program, zoo
    from nnc_py_amd.compiler import executor
    x = np.random.default_rng(6).standard_normal((batch, 3, 224, 224)).astype(np.float32)
    executor.PROJECTION_FUSION = False  # the kernels of the two-stream program, on one stream
    try:
        one = Executor(build_program(zoo.resnet18(batch=batch, seed=1), opt_level=3, branch_streams=False),
                       device=True)
    finally:
        executor.PROJECTION_FUSION = True
    one.set_input("input", x)
    one.run()
    want = one.get("output")
    one.close()
    prog = build_program(zoo.resnet18(batch=batch, seed=1), opt_level=3, branch_streams=True)
    assert len(prog.branches) == 3
    two = Executor(prog, device=True)
    two.set_input("input", x)
    two.run()
    assert caserun.same_bits(two.get("output"), want)
    two.capture()
    for _ in range(3):
        two.replay()
        runtime.sync()
        assert caserun.same_bits(two.get("output"), want)
        two.run()
        runtime.sync()
    two.close()


def test_graph_replay_matches_eager(hip):
    """A captured hipGraph replayed several times, with eager work and
    synchronisations in between, gives the eager result every time."""
    from nnc_py_amd import runtime
    from nnc_py_amd.compiler import Executor, build_program, zoo
    x = np.random.default_rng(5).standard_normal((2, 3, 224, 224)).astype(np.float32)
    ex = Executor(build_program(zoo.resnet18(batch=2, seed=1), opt_level=3), device=True)
    ex.set_input("input", x)
    ex.run()
    eager = ex.get("output")
    ex.capture()
    for _ in range(3):
        ex.replay()
        runtime.sync()
        assert caserun.same_bits(ex.get("output"), eager)
        ex.run()  # eager work between replays
        runtime.sync()
    ex.close()


def test_self_residual_block_matches_oracle(hip, oracle_lib):
    """relu(conv(h) + h) with h an intermediate, at a size with many tiles
    (batch 8, 64 channels, 56x56: 196 pixel tiles): the fused conv reads h
    as image and residual and must not write over it (the arena plan gives
    the output its own slot). GPU program vs the oracle program, O3."""
    from nnc_py_amd.compiler import Executor, build_program
    from test_compiler import _self_residual_graph
    prog = build_program(_self_residual_graph(batch=8, c=64, hw=56), opt_level=3)
    fused = [n for n in prog.order if n.op_type == "FusedConvAddRelu"]
    assert len(fused) == 1 and prog.plan.offsets[fused[0].outputs[0]] != prog.plan.offsets[fused[0].inputs[0]]
    x = np.random.default_rng(3).standard_normal((8, 64, 56, 56)).astype(np.float32)
    dev = Executor(prog, device=True)
    dev.set_input("x", x)
    dev.run()
    out = prog.graph.outputs[0]
    got = dev.get(out)
    dev.close()
    host = Executor(build_program(_self_residual_graph(batch=8, c=64, hw=56), opt_level=3), device=False,
                    lib=oracle_lib)
    host.set_input("x", x)
    host.run()
    want = host.get(out)
    bad = caserun.fp_violations(got, want, 1e-4, 1e-3)
    assert bad.size == 0, f"{bad.size} of {want.size} outside the bar"


def test_concurrent_host_threads_match_serial(hip):
    """Four host threads, each running its own ResNet-18 batch-1 program
    (O3, its own arena and input) three times while the others run: every
    output equals that program's serial result bit for bit. Each thread gets
    its own library streams and stream-K scratch on its first call, so the
    concurrent calls share nothing but the kernels (the reference's O3
    runtime calls the ops from four pthreads). Threads are started anew per
    repetition, so released per-thread states are reused too."""
    import threading
    from nnc_py_amd import runtime
    from nnc_py_amd.compiler import Executor, build_program, zoo
    n = 4
    rng = np.random.default_rng(11)
    exes, want = [], []
    for i in range(n):
        ex = Executor(build_program(zoo.resnet18(batch=1, seed=1), opt_level=3), device=True)
        ex.set_input("input", rng.standard_normal((1, 3, 224, 224)).astype(np.float32))
        ex.run()
        want.append(ex.get("output"))
        exes.append(ex)
    assert not caserun.same_bits(want[0], want[1])  # different inputs, different logits
    failures: list[str] = []
    stop = threading.Event()

    def worker(i: int, rep: int) -> None:
        try:
            if stop.is_set():
                return
            for _ in range(4):
                exes[i].run()
            runtime.sync()  # this thread's streams
            got = exes[i]._read("output")
            if runtime.last_error()[0] != 0:
                raise RuntimeError(runtime.last_error()[1])
            if not caserun.same_bits(got, want[i]):
                raise AssertionError(f"thread {i}, repetition {rep}: output differs from the serial run")
        except Exception as e:  # noqa: BLE001 - reported by the main thread
            failures.append(f"{type(e).__name__}: {e}")
            stop.set()

    for rep in range(3):
        print(f"concurrent threads: repetition {rep}", flush=True)
        threads = [threading.Thread(target=worker, args=(i, rep)) for i in range(n)]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
        assert not failures, failures[0]
    for ex in exes:
        ex.close()


def test_gap_gemm_streamed_program_matches_unfused(hip):
    """ResNet-18 batch 2 with the classifier tile-streamed from the global
    average pool (nnc_hip_gap_gemm_nt, chosen by the O3 pass when allowed)
    gives the unfused program's logits within the per-op bar (the unfused
    classifier accumulates on fp32 MFMA, the fused one in double)."""
    from nnc_py_amd.compiler import Executor, build_program, passes, zoo
    x = np.random.default_rng(8).standard_normal((2, 3, 224, 224)).astype(np.float32)
    outs = {}
    old = passes.GAP_GEMM_MAX_BATCH
    for limit in (0, 2):
        passes.GAP_GEMM_MAX_BATCH = limit
        try:
            prog = build_program(zoo.resnet18(batch=2, seed=1), opt_level=3)
        finally:
            passes.GAP_GEMM_MAX_BATCH = old
        assert (prog.calls[-1].op == "nnc_hip_gap_gemm_nt") == (limit == 2)
        ex = Executor(prog, device=True)
        ex.set_input("input", x)
        ex.run()
        outs[limit] = ex.get("output")
        ex.close()
    assert caserun.fp_violations(outs[2], outs[0], 1e-4, 1e-3).size == 0, np.abs(outs[2] - outs[0]).max()


@pytest.mark.parametrize("batch", [2, 32])
def test_conv_pool_streamed_program_matches_oracle(batch, hip, dmem, abi, oracle_lib):
    """ResNet-18 with the stem streamed into its max pool
    (nnc_hip_conv_maxpool, chosen by the O3 pass when allowed), batch 2 and
    32: the fused call against the oracle's composition on the same input at
    the per-op bar, and the logits against the unfused GPU program within the
    end-to-end bar (the two stems sum their products in different orders)."""
    from nnc_py_amd.compiler import Executor, build_program, passes, zoo
    x = np.random.default_rng(9).standard_normal((batch, 3, 224, 224)).astype(np.float32)
    old = passes.CONV_POOL_MIN_ROWS
    passes.CONV_POOL_MIN_ROWS = 1
    try:
        prog = build_program(zoo.resnet18(batch=batch, seed=1), opt_level=3)
    finally:
        passes.CONV_POOL_MIN_ROWS = old
    call = prog.calls[0]
    assert call.op == "nnc_hip_conv_maxpool"
    out_name = call.args[3][1]
    values = {"input": x, out_name: np.zeros(prog.graph.tensors[out_name].shape, np.float32)}
    for name in call.args[1:3]:
        values[name[1]] = prog.graph.tensors[name[1]].data
    case = _call_case(prog, call, values)
    got = caserun.run_case(hip, case, abi, dmem)[out_name]
    want = caserun.run_case(oracle_lib, case, abi)[out_name]
    bad = caserun.fp_violations(got, want, 1e-4, 1e-3)
    assert bad.size == 0, f"{bad.size} pooled outputs outside the bar"
    ex = Executor(prog, device=True)
    ex.set_input("input", x)
    ex.run()
    fused = ex.get("output")
    ex.close()
    ex = Executor(build_program(zoo.resnet18(batch=batch, seed=1), opt_level=3), device=True)
    ex.set_input("input", x)
    ex.run()
    plain = ex.get("output")
    ex.close()
    assert caserun.fp_violations(fused, plain, 3e-3, 1.5e-2).size == 0
