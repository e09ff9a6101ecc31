"""Shared fixtures. GPU tests carry @pytest.mark.gpu and run on an MI355X box;
everything else runs on the CPU."""

from __future__ import annotations

import ctypes
import importlib.util
import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
TESTS = Path(__file__).resolve().parent
sys.path.insert(0, str(TESTS))
sys.path.insert(0, str(TESTS / "golden"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    """Import the package directory nnc-py_amd/ as module `nnc_py_amd`."""
    if "nnc_py_amd" in sys.modules:
        return sys.modules["nnc_py_amd"]
    pkg = ROOT / "nnc-py_amd"
    spec = importlib.util.spec_from_file_location(
        "nnc_py_amd", pkg / "__init__.py", submodule_search_locations=[str(pkg)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["nnc_py_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def abi(pkg):
    from nnc_py_amd import abi as _abi
    return _abi


def _oracle_path():
    return ROOT / "oracle" / "liboracle.so"


@pytest.fixture(scope="session")
def oracle_lib(abi):
    path = _oracle_path()
    if not path.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "oracle"], check=True,
                       capture_output=True)
    return abi.bind(ctypes.CDLL(str(path)))


@pytest.fixture(scope="session")
def ref_lib(abi):
    """The reference runtime compiled from its own source (oracle/_ref); absent
    where the reference tree never was."""
    path = ROOT / "oracle" / "_ref" / "libref_ops.so"
    if not path.exists():
        pytest.skip("oracle/_ref/libref_ops.so not built (reference tree absent)")
    return abi.bind(ctypes.CDLL(str(path)))


@pytest.fixture(scope="session")
def hip(pkg):
    """libnnc_hip.so initialised on device 0 (GPU tests only). No fallback:
    a missing library fails the test."""
    from nnc_py_amd import runtime
    lib = runtime.init(0)
    yield lib
    runtime.sync()


@pytest.fixture
def dmem(hip):
    from nnc_py_amd import runtime
    runtime.clear_error()
    mem = runtime.DeviceMem()
    yield mem
    mem.release()


def load_golden():
    manifest = json.loads((TESTS / "golden" / "manifest.json").read_text())
    arrays = np.load(TESTS / "golden" / "golden.npz")
    cases = []
    for entry in manifest:
        c = dict(entry)
        c["args"] = [tuple(a) for a in entry["args"]]
        c["tensors"] = {k: arrays[f"{entry['name']}::in::{k}"] for k in entry["tensors"]}
        c["expected"] = {k: arrays[f"{entry['name']}::out::{k}"] for k in entry["outputs"]}
        cases.append(c)
    return cases


GOLDEN = load_golden()
