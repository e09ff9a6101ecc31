"""The mi355x code generator: Compiler(target="mi355x").compile() output.

CPU: file set and content (entry points, NNCB constants), and the generated
C built against a host stand-in of nnc_hip.h + the CPU oracle, whose
nnc_run() must reproduce the in-process executor bit-for-bit.
GPU: the generated C built with its own Makefile against libnnc_hip.so;
./model's printed outputs and libmodel.so's nnc_run() checked against the
oracle.
"""

from __future__ import annotations

import ctypes
import re
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import caserun

ROOT = Path(__file__).resolve().parent.parent


def _compile(tmp: Path, graph, opt=3, entry="nnc_run"):
    from nnc_py_amd.compiler.compiler import Compiler
    c = Compiler(target="mi355x", opt_level=opt)
    prog = c.compile(graph, str(tmp), entry_point=entry)
    return prog


def _lenet(batch=1):
    from nnc_py_amd.compiler import zoo
    return zoo.lenet5(batch=batch, seed=1)


def test_compiler_targets(pkg):
    from nnc_py_amd.compiler.compiler import Compiler, parse_memory_size
    with pytest.raises(NotImplementedError):
        Compiler(target="npu")
    with pytest.raises(ValueError):
        Compiler(target="tpu")
    assert parse_memory_size("256K") == 262144
    assert parse_memory_size("16MB") == 16 * 1024 * 1024
    assert parse_memory_size("1.5G") == int(1.5 * (1 << 30))
    with pytest.raises(ValueError):
        parse_memory_size("lots")


def test_generated_files_and_calls(tmp_path, pkg):
    prog = _compile(tmp_path, _lenet(), opt=3, entry="lenet_forward")
    files = {p.name for p in tmp_path.iterdir()}
    assert {"model.c", "model.h", "tensors.c", "constants.bin", "constants_loader.c",
            "test_runner.c", "Makefile"} <= files
    model_c = (tmp_path / "model.c").read_text()
    assert "nnc_conv_relu(&tensor_input" in model_c          # 5x5 conv fused with relu
    assert "nnc_maxpool2d(" in model_c and "nnc_gemm_nt(" in model_c
    assert "void nnc_run(void)" in model_c and "void lenet_forward(void)" in model_c
    header = (tmp_path / "model.h").read_text()
    assert "int nnc_load_constants(const char* path);" in header
    assert re.search(r"#define NNC_MEMORY_SIZE \d+", (tmp_path / "tensors.c").read_text())
    # Gemm+Relu is not one of the reference's fusion patterns; Flatten is an
    # alias of the pooled tensor at O3 (no call)
    assert [c.op for c in prog.calls] == [
        "nnc_conv_relu", "nnc_maxpool2d", "nnc_conv_relu", "nnc_maxpool2d",
        "nnc_gemm_nt", "nnc_relu", "nnc_gemm_nt", "nnc_relu", "nnc_gemm_nt"]


def test_nncb_constants_layout(tmp_path, pkg):
    prog = _compile(tmp_path, _lenet(), opt=1)
    blob = (tmp_path / "constants.bin").read_bytes()
    assert blob[:4] == b"NNCB"
    version, count = struct.unpack_from("<II", blob, 4)
    assert version == 1 and count == len(prog.graph.constants)
    off = 12
    for name, t in prog.graph.constants.items():
        (nlen,) = struct.unpack_from("<I", blob, off)
        sym = blob[off + 4:off + 4 + nlen - 1].decode()
        assert sym == "tensor_" + re.sub(r"[^0-9A-Za-z]+", "_", name).strip("_")
        off += 4 + nlen
        dtype, ndim = struct.unpack_from("<II", blob, off)
        off += 8
        shape = struct.unpack_from(f"<{ndim}q", blob, off)
        off += 8 * ndim
        (nbytes,) = struct.unpack_from("<Q", blob, off)
        off += 8
        assert dtype == 0 and tuple(shape) == tuple(t.shape) and nbytes == t.nbytes
        assert np.frombuffer(blob, np.float32, t.numel, off).tobytes() == t.data.tobytes()
        off += nbytes
    assert off == len(blob)


def _build_with_shim(tmp: Path) -> Path:
    inc = ROOT / "include"
    srcs = ["model.c", "tensors.c", "constants_loader.c", "test_runner.c"]
    exe = tmp / "model_host"
    cmd = ["gcc", "-std=c11", "-O1", "-D_GNU_SOURCE", "-DNNC_NO_GRAPH", f"-I{inc}", "-o", str(exe)]
    cmd += [str(tmp / s) for s in srcs] + [str(ROOT / "tests" / "host_hip_shim.c"),
                                          str(ROOT / "oracle" / "nnc_oracle.c"), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


def _parse_outputs(text: str) -> np.ndarray:
    return np.array([float(m) for m in re.findall(r"output\[\d+\] = (\S+)", text)], np.float32)


@pytest.mark.parametrize("opt", [0, 1, 3])
def test_generated_c_runs_on_the_oracle(tmp_path, pkg, oracle_lib, opt):
    from nnc_py_amd.compiler import Executor, build_program
    _compile(tmp_path, _lenet(batch=2), opt=opt)
    exe = _build_with_shim(tmp_path)
    run = subprocess.run([str(exe), str(tmp_path / "constants.bin"), "1"], capture_output=True, text=True,
                         timeout=60)
    assert run.returncode == 0, run.stderr
    got = _parse_outputs(run.stdout)
    ex = Executor(build_program(_lenet(batch=2), opt_level=opt), device=False, lib=oracle_lib)
    x = (np.arange(2 * 28 * 28, dtype=np.float32) * np.float32(0.01)).reshape(2, 1, 28, 28)
    ex.set_input("input", x)
    ex.run()
    want = ex.get("output").ravel()[:10]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)  # printed with %f


def test_generated_c_with_stream_branches_runs_on_the_oracle(tmp_path, pkg, oracle_lib, monkeypatch):
    """ResNet-18 with its downsample branches on the second stream: model.c
    calls the fork/select/join entry points inline between the node
    functions and computes what the executor computes."""
    from nnc_py_amd.compiler import Executor, build_program, executor, zoo
    monkeypatch.setattr(executor, "BRANCH_STREAMS", True)
    prog = _compile(tmp_path, zoo.resnet18(batch=1, seed=1), opt=3)
    assert len(prog.branches) == 3
    src = (tmp_path / "model.c").read_text()
    assert src.count("nnc_hip_stream_fork();") == 3 and src.count("nnc_hip_stream_join();") == 3
    assert src.count("nnc_hip_stream_select(1);") == 3 and src.count("nnc_hip_stream_select(0);") == 3
    exe = _build_with_shim(tmp_path)
    run = subprocess.run([str(exe), str(tmp_path / "constants.bin"), "1"], capture_output=True, text=True,
                         timeout=120)
    assert run.returncode == 0, run.stderr
    ex = Executor(build_program(zoo.resnet18(batch=1, seed=1), opt_level=3), device=False, lib=oracle_lib)
    ex.set_input("input", (np.arange(3 * 224 * 224, dtype=np.float32) * np.float32(0.01)).reshape(1, 3, 224, 224))
    ex.run()
    np.testing.assert_allclose(_parse_outputs(run.stdout), ex.get("output").ravel()[:10], rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("branches", [False, True])
def test_generated_c_on_gpu_make_and_run(tmp_path, hip, oracle_lib, monkeypatch, branches):
    from nnc_py_amd.compiler import Executor, build_program, executor, zoo
    monkeypatch.setattr(executor, "BRANCH_STREAMS", branches)
    _compile(tmp_path, zoo.resnet18(batch=1, seed=1), opt=3)
    subprocess.run(["make", "-C", str(tmp_path), "-j4"], check=True, capture_output=True, text=True)
    print("built generated ResNet-18 model", flush=True)
    run = subprocess.run([str(tmp_path / "model"), str(tmp_path / "constants.bin"), "3"], capture_output=True,
                         text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    got = _parse_outputs(run.stdout)
    ex = Executor(build_program(zoo.resnet18(batch=1, seed=1), opt_level=1), device=False, lib=oracle_lib)
    ex.set_input("input", (np.arange(3 * 224 * 224, dtype=np.float32) * np.float32(0.01)).reshape(1, 3, 224, 224))
    ex.run()
    want = ex.get("output").ravel()[:10]
    bad = caserun.fp_violations(got, want, 3e-3, 1.5e-2)
    assert bad.size == 0, f"generated model output {got} vs oracle {want}"


def test_generated_c_with_fused_eltwise_runs_on_the_oracle(tmp_path, pkg, oracle_lib):
    """An O3 program that is one element-wise chain: model.c hands the
    chain's inputs, steps and Clip bounds to nnc_hip_fused_eltwise as static
    arrays and computes what the executor computes."""
    from nnc_py_amd.compiler import Executor, GraphBuilder, build_program

    def chain():
        b = GraphBuilder("chain")
        x = b.input("input", (2, 3, 8, 8))
        t = b.add(b.mul(b.tanh(x), x), x)
        b.output(b.sigmoid(b.clip(t, -0.5, 0.75), out="output"))
        return b.build()
    prog = _compile(tmp_path, chain(), opt=3)
    assert [c.op for c in prog.calls] == ["nnc_hip_fused_eltwise"]
    src = (tmp_path / "model.c").read_text()
    assert "static const int" in src and "static const float" in src and "nnc_hip_fused_eltwise(" in src
    exe = _build_with_shim(tmp_path)
    run = subprocess.run([str(exe), str(tmp_path / "constants.bin"), "1"], capture_output=True, text=True,
                         timeout=60)
    assert run.returncode == 0, run.stderr
    ex = Executor(build_program(chain(), opt_level=3), device=False, lib=oracle_lib)
    ex.set_input("input", (np.arange(2 * 3 * 8 * 8, dtype=np.float32) * np.float32(0.01)).reshape(2, 3, 8, 8))
    ex.run()
    np.testing.assert_allclose(_parse_outputs(run.stdout), ex.get("output").ravel()[:10], rtol=1e-5, atol=1e-5)
