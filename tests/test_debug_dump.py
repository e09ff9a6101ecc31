"""Per-tensor debug dumps (Compiler(debug_mode=True) / Executor.run_debug) and
the dump comparison tool.

CPU: the dump format round-trips through the parser; the comparison flags a
planted mismatch at the node where it was planted; the generated debug C,
linked with the host stand-in of nnc_hip.h and the CPU oracle, writes the
same dump (names, node indices, values) as the in-process executor on the
oracle. GPU: ResNet-18 (batch 1) and the generated LeNet-5 debug build on
libnnc_hip.so, every layer compared with the oracle's dump of the same
program (the reference's allclose rule with its ResNet bar, rtol 1.5e-2 /
atol 3e-3, tests/test_common.py:545-546)."""

from __future__ import annotations

import io
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def _tools():
    from nnc_py_amd.tools import debug_compare
    return debug_compare


def test_dump_format_round_trip(tmp_path, pkg):
    dc = _tools()
    rng = np.random.default_rng(0)
    tensors = {"a": rng.standard_normal((2, 3, 4)).astype(np.float32), "b": np.float32(3.5),
               "c": np.arange(5, dtype=np.int64)}
    path = tmp_path / "dump.txt"
    with open(path, "w") as f:
        for i, (k, v) in enumerate(tensors.items()):
            dc.write_tensor(f, k, i, np.asarray(v))
    text = path.read_text()
    assert text.startswith("DEBUG_TENSOR_START a 0\nSHAPE 3\nDIM 0 2\nDIM 1 3\nDIM 2 4\nDATA_START\n")
    got = dc.DebugOutputParser(path).parse()
    assert [got[k]["node_idx"] for k in "abc"] == [0, 1, 2]
    np.testing.assert_allclose(got["a"]["data"], tensors["a"], atol=5e-7)  # printed with %f
    assert got["b"]["data"].shape == () and got["b"]["data"] == np.float32(3.5)
    np.testing.assert_array_equal(got["c"]["data"], np.arange(5, dtype=np.float32))


def test_compare_finds_the_first_mismatching_node(pkg):
    dc = _tools()
    rng = np.random.default_rng(1)
    ref = {f"t{i}": {"node_idx": i, "data": rng.standard_normal(8).astype(np.float32)} for i in range(4)}
    nnc = {k: dict(v, data=v["data"].copy()) for k, v in ref.items()}
    nnc["t2"]["data"][3] += 0.5
    nnc["t3"]["data"][0] += 1.0
    nnc["t1"]["data"] = nnc["t1"]["data"].reshape(2, 4)
    del nnc["t0"]
    res = dc.compare_outputs(nnc, ref)
    assert res["missing_in_nnc"] == ["t0"] and [m["tensor"] for m in res["shape_mismatch"]] == ["t1"]
    assert [m["tensor"] for m in res["mismatched"]] == ["t2", "t3"]
    assert res["first_mismatch"]["tensor"] == "t2" and abs(res["first_mismatch"]["max_diff"] - 0.5) < 1e-6
    out = io.StringIO()
    assert dc.DebugComparator.print_report(res, out) == 1 and "first mismatching node: 2" in out.getvalue()


def _lenet(batch=1):
    from nnc_py_amd.compiler import zoo
    return zoo.lenet5(batch=batch, seed=1)


def _oracle_dump(path, graph, opt, oracle_lib, x):
    from nnc_py_amd.compiler import Executor, build_program
    ex = Executor(build_program(graph, opt_level=opt), device=False, lib=oracle_lib)
    ex.set_input("input", x)
    ex.run_debug(path)


@pytest.mark.parametrize("opt", [1, 3])
def test_generated_debug_build_matches_the_executor_dump(tmp_path, pkg, oracle_lib, opt):
    from nnc_py_amd.compiler.compiler import Compiler
    Compiler(target="mi355x", opt_level=opt, debug_mode=True).compile(_lenet(), str(tmp_path))
    model_c = (tmp_path / "model.c").read_text()
    assert "nnc_hip_debug_dump(" in model_c and "nnc_hip_graph_begin" not in model_c
    assert "FILE* debug_file = NULL;" in (tmp_path / "test_runner.c").read_text()
    inc = ROOT / "include"
    exe = tmp_path / "model_dbg"
    srcs = [str(tmp_path / s) for s in ("model.c", "tensors.c", "constants_loader.c", "test_runner.c")]
    subprocess.run(["gcc", "-std=c11", "-O1", "-D_GNU_SOURCE", f"-I{inc}", "-o", str(exe), *srcs,
                    str(ROOT / "tests" / "host_hip_shim.c"), str(ROOT / "oracle" / "nnc_oracle.c"), "-lm"],
                   check=True, capture_output=True, text=True)
    run = subprocess.run([str(exe), str(tmp_path / "constants.bin")], capture_output=True, text=True, timeout=60,
                         cwd=tmp_path)
    assert run.returncode == 0, run.stderr
    x = (np.arange(28 * 28, dtype=np.float32) * np.float32(0.01)).reshape(1, 1, 28, 28)
    _oracle_dump(tmp_path / "ref.txt", _lenet(), opt, oracle_lib, x)
    dc = _tools()
    got = dc.DebugOutputParser(tmp_path / "nnc_debug_output.txt").parse()
    want = dc.DebugOutputParser(tmp_path / "ref.txt").parse()
    assert list(got) == list(want) and len(got) >= 8
    assert [v["node_idx"] for v in got.values()] == [v["node_idx"] for v in want.values()]
    res = dc.compare_outputs(got, want, rtol=0.0, atol=0.0)  # same arithmetic, same printing
    assert len(res["matched"]) == len(want), res


@pytest.mark.gpu
def test_resnet18_layerwise_against_oracle(tmp_path, hip, oracle_lib):
    from nnc_py_amd.compiler import Executor, build_program, zoo
    x = np.random.default_rng(0).standard_normal((1, 3, 224, 224)).astype(np.float32)
    prog = build_program(zoo.resnet18(batch=1, seed=1), opt_level=3)
    ex = Executor(prog, device=True)
    ex.set_input("input", x)
    ex.run_debug(tmp_path / "gpu.txt")
    ex.close()
    print("dumped ResNet-18 on the GPU", flush=True)
    _oracle_dump(tmp_path / "ref.txt", zoo.resnet18(batch=1, seed=1), 3, oracle_lib, x)
    dc = _tools()
    res = dc.DebugComparator(tmp_path / "gpu.txt", tmp_path / "ref.txt", rtol=1.5e-2, atol=3e-3).compare()
    assert not res["mismatched"] and not res["shape_mismatch"] and not res["missing_in_nnc"], res
    assert len(res["matched"]) == len(prog.order)  # every node's output (the O3 program has 19 nodes)


@pytest.mark.gpu
def test_generated_debug_build_on_gpu(tmp_path, hip, oracle_lib):
    from nnc_py_amd.compiler.compiler import Compiler
    Compiler(target="mi355x", opt_level=3, debug_mode=True).compile(_lenet(), str(tmp_path))
    subprocess.run(["make", "-C", str(tmp_path), "-j4", "model"], check=True, capture_output=True, text=True)
    print("built the generated LeNet-5 debug model", flush=True)
    run = subprocess.run([str(tmp_path / "model"), str(tmp_path / "constants.bin")], capture_output=True,
                         text=True, timeout=120, cwd=tmp_path)
    assert run.returncode == 0, run.stderr
    x = (np.arange(28 * 28, dtype=np.float32) * np.float32(0.01)).reshape(1, 1, 28, 28)
    _oracle_dump(tmp_path / "ref.txt", _lenet(), 3, oracle_lib, x)
    dc = _tools()
    res = dc.DebugComparator(tmp_path / "nnc_debug_output.txt", tmp_path / "ref.txt").compare()
    assert not res["mismatched"] and not res["shape_mismatch"] and not res["missing_in_nnc"], res
