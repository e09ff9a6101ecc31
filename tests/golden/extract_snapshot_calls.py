"""Extract the nnc_* call sequence of the reference's codegen snapshots into a
data fixture (tests/golden/snapshot_calls.json).

Source (read as text, in the container that holds the reference tree):
  tests/__snapshots__/test_snapshots_resnet18.ambr (model.c section)
  tests/__snapshots__/test_snapshots_lenet5.ambr   (model.c section)
Each entry: node function, nnc_* entry point, argument list (tensor symbols
as written, numbers as numbers).

Run:  python tests/golden/extract_snapshot_calls.py
"""

from __future__ import annotations

import json
import re
from pathlib import Path

REF = Path("/root/reference/tests/__snapshots__")
OUT = Path(__file__).resolve().parent / "snapshot_calls.json"

_NODE = re.compile(r"^\s*void (node_\w+)\(void\) \{\s*\n\s*(nnc_\w+)\((.*)\);", re.M)


def _arg(a: str):
    a = a.strip()
    if a.startswith("&"):
        return a[1:]
    if a == "NULL":
        return None
    if a.endswith("f") and re.match(r"^-?[\d.]+(e-?\d+)?f$", a):
        return float(a[:-1])
    return int(a)


def extract(path: Path) -> list[dict]:
    text = path.read_text()
    section = text.split("// model.h")[0]  # the model.c part of the codegen snapshot
    calls = []
    for node, op, args in _NODE.findall(section):
        calls.append({"node": node, "op": op, "args": [_arg(a) for a in args.split(",")]})
    return calls


def main():
    data = {"resnet18": extract(REF / "test_snapshots_resnet18.ambr"),
            "lenet5": extract(REF / "test_snapshots_lenet5.ambr")}
    OUT.write_text(json.dumps(data, indent=1) + "\n")
    print({k: len(v) for k, v in data.items()})


if __name__ == "__main__":
    main()
