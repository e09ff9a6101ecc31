"""Write the golden vectors: every case of cases.py run through the REFERENCE
runtime (runtime/x86/ops.c compiled by oracle/Makefile into
oracle/_ref/libref_ops.so, in the container that holds the reference tree).

Outputs (committed fixtures, data only):
  tests/golden/golden.npz     inputs "<case>::in::<key>" and reference outputs
                              "<case>::out::<key>"
  tests/golden/manifest.json  call description of every case

nnc_matmul_relu has no reference definition (the reference code generator
emits the call, no reference runtime defines it); its expected value is the
reference nnc_matmul followed by max(0, x).

Run:  make -C oracle ref && python tests/golden/make_golden.py
"""

from __future__ import annotations

import ctypes
import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE))

import caserun  # noqa: E402
import cases  # noqa: E402


def load_abi():
    spec = importlib.util.spec_from_file_location("nnc_abi", ROOT / "nnc-py_amd" / "abi.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main():
    abi = load_abi()
    ref_path = ROOT / "oracle" / "_ref" / "libref_ops.so"
    if not ref_path.exists():
        sys.exit(f"{ref_path} missing: run `make -C oracle ref` where the reference tree exists")
    ref = abi.bind(ctypes.CDLL(str(ref_path)))
    arrays = {}
    manifest = []
    for c in cases.all_cases():
        if c["op"] in abi.NOT_IN_REFERENCE:
            base = dict(c, op="nnc_matmul", args=[a for a in c["args"] if a[0] != "null"])
            res = caserun.run_case(ref, base, abi)
            res = {k: np.where(v > 0, v, np.float32(0)).astype(v.dtype) for k, v in res.items()}
        else:
            res = caserun.run_case(ref, c, abi)
        for k, v in c["tensors"].items():
            arrays[f"{c['name']}::in::{k}"] = v
        for k, v in res.items():
            arrays[f"{c['name']}::out::{k}"] = v
        entry = {k: v for k, v in c.items() if k != "tensors"}
        entry["args"] = [list(a) for a in c["args"]]
        entry["tensors"] = {k: {"shape": list(v.shape), "dtype": v.dtype.name}
                            for k, v in c["tensors"].items()}
        manifest.append(entry)
    np.savez_compressed(HERE / "golden.npz", **arrays)
    (HERE / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    size = (HERE / "golden.npz").stat().st_size
    print(f"{len(manifest)} cases, golden.npz {size / 1e6:.2f} MB")


if __name__ == "__main__":
    main()
