"""Layer-by-layer comparison of debug dumps.

A program compiled with Compiler(debug_mode=True) writes every node's output
after the node runs, in the reference's text format (emitted by
src/nnc_py/codegen/x86_emitters/model_source.py:136-184, 297-428; read by
src/nnc_py/tools/debug_compare.py:17-106):

    DEBUG_TENSOR_START <name> <node_idx>
    SHAPE <ndim>
    DIM <i> <extent>
    DATA_START
    <one %f value per line>
    DATA_END
    DEBUG_TENSOR_END <name>

The generated C does it through nnc_hip_debug_dump (libnnc_hip.so) into
nnc_debug_output.txt; Executor.run_debug() writes the same file from Python,
for any implementation of the ABI the executor is bound to.

The reference compares such a dump with ONNX Runtime; here two dumps are
compared with each other - e.g. the mi355x program's against the dump of the
reference's x86 build of the same model (same tensor names, same format),
or against any other run of the program. The tolerance rule is numpy's
allclose(nnc, ref, rtol, atol), as the reference's DebugComparator, with the
same defaults (rtol 1e-4, atol 1e-5).

    python -m nnc_py_amd.tools.debug_compare nnc_debug_output.txt reference_dump.txt
"""

from __future__ import annotations

import sys
from pathlib import Path
from typing import Any, TextIO

import numpy as np


def write_tensor(f: TextIO, name: str, node_idx: int, arr: np.ndarray) -> None:
    """One tensor in the dump format (values converted to float32, %f)."""
    a = np.asarray(arr)
    f.write(f"DEBUG_TENSOR_START {name} {node_idx}\n")
    f.write(f"SHAPE {a.ndim}\n")
    for i, d in enumerate(a.shape):
        f.write(f"DIM {i} {int(d)}\n")
    f.write("DATA_START\n")
    vals = a.astype(np.float32).ravel().astype(np.float64)
    f.write("".join(f"{v:f}\n" for v in vals))
    f.write("DATA_END\n")
    f.write(f"DEBUG_TENSOR_END {name}\n\n")


class DebugOutputParser:
    """Reads a dump into {name: {"node_idx", "ndim", "shape", "data"}}."""

    def __init__(self, debug_file: str | Path):
        self.debug_file = Path(debug_file)
        self.outputs: dict[str, dict[str, Any]] = {}

    def parse(self) -> dict[str, dict[str, Any]]:
        self.outputs = {}
        cur: dict[str, Any] | None = None
        values: list[float] = []
        in_data = False
        with open(self.debug_file) as f:
            for raw in f:
                line = raw.strip()
                if not line:
                    continue
                if line.startswith("DEBUG_TENSOR_START"):
                    _, name, idx = line.split()
                    cur = {"name": name, "node_idx": int(idx), "ndim": 0, "shape": []}
                    in_data = False
                elif cur is None:
                    continue
                elif line.startswith("SHAPE"):
                    cur["ndim"] = int(line.split()[1])
                elif line.startswith("DIM"):
                    cur["shape"].append(int(line.split()[2]))
                elif line == "DATA_START":
                    in_data, values = True, []
                elif line == "DATA_END":
                    in_data = False
                    data = np.array(values, np.float32)
                    if cur["ndim"] == 0 and data.size == 1:
                        data = data.reshape(())
                    elif cur["shape"] and all(d >= 0 for d in cur["shape"]) and \
                            int(np.prod(cur["shape"])) == data.size:
                        data = data.reshape(cur["shape"])
                    cur["data"] = data
                    self.outputs[cur["name"]] = cur
                elif line.startswith("DEBUG_TENSOR_END"):
                    cur = None
                elif in_data:
                    values.append(float(line))
        return self.outputs


def compare_outputs(nnc: dict[str, dict[str, Any]], ref: dict[str, dict[str, Any]], rtol: float = 1e-4,
                    atol: float = 1e-5) -> dict[str, Any]:
    """Tensor by tensor: matched / mismatched (max |diff|, node) / shape
    mismatches / names present on one side only; `first_mismatch` is the
    mismatching tensor with the lowest node index - where the two runs part."""
    res: dict[str, Any] = {"matched": [], "mismatched": [], "shape_mismatch": [], "missing_in_nnc": [],
                           "missing_in_reference": []}
    for name in sorted(set(nnc) | set(ref), key=lambda n: (nnc.get(n) or ref.get(n))["node_idx"]):
        a, b = nnc.get(name), ref.get(name)
        if a is None:
            res["missing_in_nnc"].append(name)
            continue
        if b is None:
            res["missing_in_reference"].append(name)
            continue
        x, y = np.asarray(a["data"]), np.asarray(b["data"])
        if list(x.shape) != list(y.shape):
            res["shape_mismatch"].append({"tensor": name, "nnc_shape": list(x.shape), "reference_shape": list(y.shape)})
            continue
        if np.allclose(x, y, rtol=rtol, atol=atol, equal_nan=True):
            res["matched"].append(name)
        else:
            diff = np.abs(x.astype(np.float64) - y.astype(np.float64))
            res["mismatched"].append({"tensor": name, "node_idx": a["node_idx"],
                                      "max_diff": float(np.nanmax(diff)) if diff.size else 0.0})
    res["first_mismatch"] = min(res["mismatched"], key=lambda m: m["node_idx"]) if res["mismatched"] else None
    return res


class DebugComparator:
    """Compare two dump files (the reference's DebugComparator, with a dump
    instead of ONNX Runtime on the reference side)."""

    def __init__(self, nnc_debug_file: str | Path, reference_dump: str | Path, rtol: float = 1e-4,
                 atol: float = 1e-5):
        self.rtol, self.atol = rtol, atol
        self.nnc_outputs = DebugOutputParser(nnc_debug_file).parse()
        self.reference_outputs = DebugOutputParser(reference_dump).parse()

    def compare(self) -> dict[str, Any]:
        return compare_outputs(self.nnc_outputs, self.reference_outputs, self.rtol, self.atol)

    @staticmethod
    def print_report(results: dict[str, Any], out: TextIO = sys.stdout) -> int:
        total = len(results["matched"]) + len(results["mismatched"]) + len(results["shape_mismatch"])
        w = out.write
        w("=" * 60 + "\nNNC (mi355x) vs reference dump\n" + "=" * 60 + "\n")
        w(f"Total tensors compared: {total}\n  matched: {len(results['matched'])}\n"
          f"  mismatched: {len(results['mismatched'])}\n  shape mismatch: {len(results['shape_mismatch'])}\n"
          f"  missing in nnc: {len(results['missing_in_nnc'])}\n"
          f"  missing in reference: {len(results['missing_in_reference'])}\n")
        for m in results["mismatched"]:
            w(f"  mismatch {m['tensor']} (node {m['node_idx']}, max diff {m['max_diff']:.6g})\n")
        for m in results["shape_mismatch"]:
            w(f"  shape {m['tensor']}: nnc {m['nnc_shape']} vs reference {m['reference_shape']}\n")
        if results["first_mismatch"]:
            w(f"first mismatching node: {results['first_mismatch']['node_idx']} "
              f"({results['first_mismatch']['tensor']})\n")
        w("=" * 60 + "\n")
        return 0 if not results["mismatched"] and not results["shape_mismatch"] else 1


def compare_debug_output(nnc_debug_file: str | Path, reference_dump: str | Path, rtol: float = 1e-4,
                         atol: float = 1e-5) -> int:
    """Compare, print the report; 0 when every common tensor matches."""
    comp = DebugComparator(nnc_debug_file, reference_dump, rtol, atol)
    return comp.print_report(comp.compare())


def main(argv: list[str] | None = None) -> int:
    import argparse
    ap = argparse.ArgumentParser(description="compare two nnc debug dumps tensor by tensor")
    ap.add_argument("nnc_debug_file")
    ap.add_argument("reference_dump")
    ap.add_argument("--rtol", type=float, default=1e-4)
    ap.add_argument("--atol", type=float, default=1e-5)
    a = ap.parse_args(argv)
    return compare_debug_output(a.nnc_debug_file, a.reference_dump, a.rtol, a.atol)


if __name__ == "__main__":
    sys.exit(main())
