"""Write costmodel_mi355x.json: measured MI355X kernel durations that pin the
cost-model runtime (libnnc_costmodel.so).

Input: rocprofv3 kernel traces of libnnc_hip.so running the O3 programs of
ResNet-18 (batch 1, 8, 32) and the transformer encoder (batch 8, sequence
128) - one eager run, three graph replays and 20 timed replays each - and the
graph-replay milliseconds per step that the same script prints when it runs
without the profiler on the same machine (kernel tracing stalls graph
replays between kernels - up to hundreds of microseconds - while the traced
kernel durations match the untraced ones):

    rocprofv3 --kernel-trace --output-format csv -d <dir>/<cfg> -o trace -- \\
        python3 tests/golden/costmodel_trace_run.py <cfg>
    python3 tests/golden/costmodel_trace_run.py <cfg>      # ms/step

Output per configuration: the replayed step time, and per kernel (demangled
name without template arguments) the launches per step and the median
duration over the timed replays (avg_us: the mean of those medians over the
kernel's launches in one step).

    python tests/golden/make_costmodel_fixture.py <dir> r18_b1=0.2661 r18_b8=0.6063 r18_b32=1.3255 tf_b8=0.2260
"""

from __future__ import annotations

import csv
import json
import re
import statistics
import sys
from pathlib import Path

RUNS = 24  # eager + 3 warm-up replays + 20 timed replays
TIMED = 20


def kernel_family(name: str) -> str:
    m = re.match(r"(?:void )?(?:nnc::)?(\w+)", name)
    return m.group(1) if m else name


def main(trace_dir: str, *steps: str) -> None:
    out = {}
    for item in steps:
        cfg, ms = item.split("=")
        rows = list(csv.DictReader(open(Path(trace_dir) / cfg / "trace_kernel_trace.csv")))
        rows = [r for r in rows if not r["Kernel_Name"].startswith("__amd")]
        rows.sort(key=lambda r: int(r["Start_Timestamp"]))
        assert len(rows) % RUNS == 0, (cfg, len(rows))
        per = len(rows) // RUNS
        tail = rows[-TIMED * per:]
        fams: dict[str, list] = {}
        for i in range(per):
            durs = [(int(tail[i + k * per]["End_Timestamp"]) - int(tail[i + k * per]["Start_Timestamp"])) / 1e3
                    for k in range(TIMED)]
            fams.setdefault(kernel_family(tail[i]["Kernel_Name"]), []).append(statistics.median(durs))
        out[cfg] = {"step_us": round(float(ms) * 1e3, 1),
                    "kernels": {f: {"launches": len(d), "avg_us": round(statistics.mean(d), 2)}
                                for f, d in sorted(fams.items())}}
    Path(__file__).with_name("costmodel_mi355x.json").write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main(*sys.argv[1:])
