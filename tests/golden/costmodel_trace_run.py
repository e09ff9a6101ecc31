"""One traced program run for make_costmodel_fixture.py: builds the O3
program of a configuration (r18_b1, r18_b8, r18_b32: ResNet-18 at that
batch; tf_b8: the transformer encoder at batch 8, sequence 128), runs it
eagerly once, captures it as a hipGraph, replays it 3 times and then 20
timed times, and prints the replayed milliseconds per step. Run under
`rocprofv3 --kernel-trace --output-format csv -d <dir>/<cfg> -o trace --`."""

from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import conftest  # noqa: E402

conftest.load_package()
from nnc_py_amd import runtime  # noqa: E402
from nnc_py_amd.compiler import Executor, build_program, zoo  # noqa: E402


def main(cfg: str, reps: int = 20) -> None:
    runtime.init(0)
    kind, b = cfg.split("_b")
    g = zoo.resnet18(batch=int(b), seed=1) if kind == "r18" else zoo.transformer_encoder(batch=int(b), seq=128)
    prog = build_program(g, opt_level=3)
    name = prog.graph.inputs[0]
    ex = Executor(prog, device=True)
    ex.set_input(name, np.random.default_rng(0).standard_normal(prog.graph.tensors[name].shape).astype(np.float32))
    ex.run()
    runtime.sync()
    ex.capture()
    for _ in range(3):
        ex.replay()
    runtime.sync()
    t = time.perf_counter()
    for _ in range(reps):
        ex.replay()
    runtime.sync()
    print(f"{cfg} ms/step {(time.perf_counter() - t) / reps * 1e3:.4f} calls {len(prog.calls)}", flush=True)
    ex.close()


if __name__ == "__main__":
    main(sys.argv[1])
