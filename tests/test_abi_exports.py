"""The C-ABI libraries load and export what include/*.h declares (CPU only:
no HIP call is made, the library is only dlopen'ed)."""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
INCLUDE = ROOT / "include"


def test_signature_table_matches_header(abi):
    declared = set(abi.declared_symbols(INCLUDE / "nnc_ops.h"))
    assert declared == set(abi.SIGNATURES), declared ^ set(abi.SIGNATURES)


def test_reference_abi_is_covered(abi):
    """Every entry point of the reference ABI (runtime/include/nnc_ops.h) is in
    our header; the only addition is the emitted-but-undefined matmul_relu."""
    ref_names = {n for n in abi.SIGNATURES if n not in abi.NOT_IN_REFERENCE}
    assert len(ref_names) == 55


def test_hip_library_exports_every_declared_symbol(abi, pkg):
    from nnc_py_amd import runtime
    if not runtime.LIB_PATH.exists():
        pytest.fail("libnnc_hip.so is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(runtime.LIB_PATH))
    missing = []
    for header in sorted(INCLUDE.glob("*.h")):
        if header.name == "nnc_costmodel.h":  # libnnc_costmodel.so's own queries (tests/test_costmodel.py)
            continue
        for name in abi.declared_symbols(header):
            if not hasattr(lib, name):
                missing.append(f"{header.name}:{name}")
    assert not missing, missing


def test_hip_header_declares_the_runtime_table(abi, pkg):
    from nnc_py_amd import runtime
    declared = set(abi.declared_symbols(INCLUDE / "nnc_hip.h"))
    assert declared == set(runtime._HIP_SIGNATURES), declared ^ set(runtime._HIP_SIGNATURES)


def test_oracle_exports_every_op(abi, oracle_lib):
    for name in abi.SIGNATURES:
        assert hasattr(oracle_lib, name), name


def test_product_does_not_link_the_oracle(pkg):
    """libnnc_hip.so must not depend on or embed the CPU oracle."""
    from nnc_py_amd import runtime
    data = runtime.LIB_PATH.read_bytes()
    assert b"liboracle" not in data and b"libref_ops" not in data


def test_oracle_internal_calls_never_reach_the_hip_library(pkg, oracle_lib):
    """The oracle's composed entry points (nnc_matmul_relu,
    nnc_hip_conv_add_relu) call its own nnc_conv / nnc_matmul / nnc_add_relu /
    nnc_relu. In a GPU test process libnnc_hip.so exports the same names; if
    those calls bound to it they would launch GPU kernels on host pointers.
    Both libraries are loaded here as a GPU test would (the HIP library even
    with RTLD_GLOBAL), with eager binding, and the dynamic linker's binding
    log must show no oracle reference resolved into libnnc_hip.so. No GPU call
    is made."""
    import os
    import subprocess
    import sys
    from nnc_py_amd import runtime
    if not runtime.LIB_PATH.exists():
        pytest.fail("libnnc_hip.so is not built: run __graft_entry__.build()")
    oracle = ROOT / "oracle" / "liboracle.so"
    code = (f"import ctypes; ctypes.CDLL({str(runtime.LIB_PATH)!r}, mode=ctypes.RTLD_GLOBAL); "
            f"ctypes.CDLL({str(oracle)!r})")
    env = dict(os.environ, LD_DEBUG="bindings", LD_BIND_NOW="1")
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr[-2000:]
    bad = [l for l in res.stderr.splitlines()
           if "liboracle.so" in l.split(" to ")[0] and "libnnc_hip.so" in l.split(" to ")[-1]]
    assert not bad, bad[:5]
