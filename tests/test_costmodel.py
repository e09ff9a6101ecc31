"""The cost-model runtime (libnnc_costmodel.so) against MI355X measurements.

The reference's runtime/x86/costmodel.c replaces the kernels with a timing
trace (tests: its summary lines and per-op trace, NNC_RUNTIME_IMPL=costmodel
in the generated Makefile, codegen/x86_emitters/build_files.py:50-81). Here
the model must also agree with the GPU it stands for:

- the kernels it prices for a program are the kernels libnnc_hip.so
  launches: per kernel family, the launches per step equal the counts in a
  rocprofv3 trace of the same program on MI355X (tests/golden/
  costmodel_mi355x.json, made by tests/golden/make_costmodel_fixture.py);
- its step time is within 25% of the measured graph-replay step, and each
  kernel family's average launch within 35% of the measured one.
On the GPU, the model's per-kernel table equals libnnc_hip.so's own
profiling table name for name and launch for launch.
"""

from __future__ import annotations

import json
import os
import re
import subprocess

import pytest

from conftest import ROOT

FIXTURE = json.loads((ROOT / "tests" / "golden" / "costmodel_mi355x.json").read_text())

# the model's kernel names (those of libnnc_hip.so's profiling table) by the
# device kernel that runs them
FAMILY = [
    (r"conv_stem_rows_", "conv_stem_k"),
    (r"conv_stem_pool_w", "conv_stem_pool_k"),
    (r"conv_igemm_.*_dma$", "conv_dma_k"),
    (r"conv_ws_32x32_", "conv_ws_k"),
    (r"conv_igemm_", "conv_streamk_k"),
    (r"conv_streamk_fixup$", "conv_fixup_k"),
    (r"gemm_dma_", "gemm_dma_k"),
    (r"gemm_ws_32x32_", "gemm_ws_k"),
    (r"attention16_d64$", "attention16_k"),
    (r"attention32_d32$", "attention_k"),
    (r"gemm_mfma_", "gemm_streamk_k"),
    (r"gemm_streamk_fixup$", "gemm_fixup_k"),
    (r"dot_rows_", "dot_k"),
    (r"gemm_skinny_nt_", "gemm_skinny_nt_k"),
    (r"nnc_hip_add_layernorm$", "layernorm_rows_v4_k"),
    (r"nnc_hip_scaled_softmax$", "softmax_rows_v4_k"),
    (r"nnc_hip_transpose_slice$", "permute_slice_k"),
    (r"nnc_hip_fused_eltwise$", "fused_eltwise_vec4_k"),
    (r"nnc_maxpool2d$", "maxpool3s2_v4_k"),
    (r"nnc_avgpool2d_global$", "global_avgpool_k"),
    (r"nnc_(add|sub|mul|div)(_relu|_sigmoid)?$", "binary_vec4_k"),
    (r"nnc_softmax$", "softmax_rows_v4_k"),
    (r"nnc_layernorm$", "layernorm_rows_v4_k"),
    (r"nnc_transpose$", "transpose"),
    (r"nnc_(split|concat)$", "slab_copy_k"),
]


def _family(name: str) -> str:
    for pat, fam in FAMILY:
        if re.match(pat, name):
            return fam
    return name


def _program(cfg: str):
    from nnc_py_amd.compiler import build_program, zoo
    kind, b = cfg.split("_b")
    g = zoo.resnet18(batch=int(b), seed=1) if kind == "r18" else zoo.transformer_encoder(batch=int(b), seq=128)
    return build_program(g, opt_level=3)


# device kernels that one launch name of libnnc_hip.so stands for
MERGED = {"permute_k": "transpose", "transpose2d_k": "transpose",
          "conv_fixup_split_k": "conv_fixup_k"}  # both "conv_streamk_fixup"


def _measured_families(cfg: str) -> dict:
    fams: dict[str, dict] = {}
    for name, k in FIXTURE[cfg]["kernels"].items():
        fam = MERGED.get(name, name)
        f = fams.setdefault(fam, {"launches": 0, "us": 0.0})
        f["launches"] += k["launches"]
        f["us"] += k["launches"] * k["avg_us"]
    return fams


@pytest.fixture(scope="module")
def cm(pkg):
    from nnc_py_amd import costmodel
    return costmodel


def test_exports_every_declared_symbol(cm):
    lib = cm.load()
    for header in ("nnc_ops.h", "nnc_hip.h", "nnc_costmodel.h"):
        text = (ROOT / "include" / header).read_text()
        names = set(re.findall(r"^\w[\w\s\*]*?\b(nnc_\w+)\s*\(", text, re.M))
        missing = [n for n in sorted(names) if not hasattr(lib, n)]
        assert not missing, (header, missing)


@pytest.mark.parametrize("cfg", sorted(FIXTURE))
def test_model_launches_the_librarys_kernels_and_tracks_their_time(cm, cfg):
    est = cm.estimate(_program(cfg))
    model: dict[str, dict] = {}
    for k in est.kernels:
        f = model.setdefault(_family(k.name), {"launches": 0, "us": 0.0})
        f["launches"] += k.launches
        f["us"] += k.us
    meas = _measured_families(cfg)
    assert {f: v["launches"] for f, v in model.items()} == {f: v["launches"] for f, v in meas.items()}
    step = FIXTURE[cfg]["step_us"]
    assert abs(est.step_us / step - 1) <= 0.25, (cfg, est.step_us, step)
    for fam, v in meas.items():
        want = v["us"] / v["launches"]
        got = model[fam]["us"] / model[fam]["launches"]
        assert abs(got / want - 1) <= 0.35, (cfg, fam, got, want)


def test_second_stream_overlaps_on_the_timeline(cm):
    """Forked branches run side by side: the two-stream program's time is
    below the sum of its kernels and not below the longer stream."""
    from nnc_py_amd.compiler import build_program, executor, zoo
    executor.PROJECTION_FUSION = False  # the same kernels as the two-stream program
    try:
        one = cm.estimate(build_program(zoo.resnet18(batch=1, seed=1), opt_level=3, branch_streams=False))
    finally:
        executor.PROJECTION_FUSION = True
    two = cm.estimate(build_program(zoo.resnet18(batch=1, seed=1), opt_level=3, branch_streams=True))
    total = sum(k.us for k in two.kernels)
    assert two.step_us < total and abs(total - one.step_us) < 1e-6
    assert two.step_us < one.step_us


def test_generated_program_links_the_cost_model(tmp_path, pkg):
    """`make run-costmodel`: the generated program runs on the timing model
    unchanged and prints the per-kernel trace and the summary."""
    from nnc_py_amd.compiler import zoo
    from nnc_py_amd.compiler.compiler import Compiler
    Compiler(target="mi355x", opt_level=3).compile(zoo.lenet5(batch=2, seed=1), str(tmp_path))
    env = {k: v for k, v in os.environ.items() if k != "NNC_COSTMODEL_QUIET"}
    run = subprocess.run(["make", "-C", str(tmp_path), "run-costmodel"], capture_output=True, text=True, timeout=120,
                         env=env)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "[costmodel] #1 op=" in run.stdout and "[costmodel] summary kernels=" in run.stdout
    assert "kernel=conv_igemm_" in run.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", ["r18_b1", "r18_b32", "tf_b8"])
def test_model_table_equals_the_librarys_profile(hip, cm, cfg):
    from nnc_py_amd import runtime
    from nnc_py_amd.compiler import Executor
    import numpy as np
    prog = _program(cfg)
    ex = Executor(prog, device=True)
    name = prog.graph.inputs[0]
    ex.set_input(name, np.zeros(prog.graph.tensors[name].shape, np.float32))
    ex.run()  # first call: one-time set-up launches
    runtime.sync()
    runtime.profile_reset()
    runtime.profile_enable(True)
    ex.run()
    table = runtime.profile_table()
    runtime.profile_enable(False)
    ex.close()
    got = {r["name"]: r["launches"] for r in table}
    est = cm.estimate(_program(cfg))
    assert {k.name: k.launches for k in est.kernels} == got
