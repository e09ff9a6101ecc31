#!/usr/bin/env python3
"""ResNet-18 fp32 inference throughput on one MI355X through libnnc_hip.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one nnc_run() of ResNet-18 (BatchNorm folded) over a batch of 32
synthetic 3x224x224 images: the O3 program (conv+relu and add+relu fused,
specialised conv entry points, constant FC weight in [N, K]) lowered to nnc_*
calls, its activations and weights in one HBM arena, replayed as one
hipGraph per step. Inputs are resident in HBM before timing starts.

Printed as one JSON line (rank 0): images/s at batch 32 (value), batch 1 as
an extra figure, the roofline of the dominant kernel measured live from the
library's per-launch hipEvent table, a per-kernel table, and the reference
CPU runtime timed on this host as a baseline.

HBM traffic of the dominant kernel (roofline.traffic) comes from two
`rocprofv3 --pmc` child runs of this script in --pmc-child mode (FETCH_SIZE,
then WRITE_SIZE), each scaled by what the same counter reads for a plain
device copy of known size run in the same child; --no-traffic skips them.
"""

from __future__ import annotations

import argparse
import csv
import ctypes
import importlib.util
import json
import os
import platform
import re
import shutil
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
METRIC = "ResNet-18 fp32 images/s (b1,b32) on 1 GPU; per-op % HBM/MFMA roofline"
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_FP32_MFMA_TF = 157.3  # MI355X dense fp32 matrix
# kernel-table names of the MFMA kernels (their work is priced in FLOP)
MFMA_KERNELS = ("conv_igemm", "conv_stem", "conv_ws", "gemm_mfma", "gemm_dma", "gemm_skinny", "gemm_ws", "attention")


def load_package():
    if "nnc_py_amd" in sys.modules:
        return sys.modules["nnc_py_amd"]
    pkg = ROOT / "nnc-py_amd"
    spec = importlib.util.spec_from_file_location("nnc_py_amd", pkg / "__init__.py",
                                                  submodule_search_locations=[str(pkg)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["nnc_py_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def timed_steps(ex, steps: int, warmup: int, graph: bool, runtime) -> float:
    """Seconds for `steps` nnc_run() after `warmup`; synchronised both sides."""
    for _ in range(warmup):
        ex.run()
    runtime.sync()
    if graph:
        ex.capture()
        ex.replay()
        runtime.sync()
    step = ex.replay if graph else ex.run
    runtime.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    runtime.sync()
    return time.perf_counter() - t0


def latency_samples(ex, iters: int, warmup: int, graph: bool, runtime) -> dict:
    """The reference harness's measurement shape (benchmarks/cases.py:23-31:
    5 warmup + 20 measured runs; benchmarks/harness.py:139-161: mean, p50
    and p95 by nearest rank): each step timed on its own, from its launch
    to the end of a synchronisation, in milliseconds."""
    for _ in range(warmup):
        ex.replay() if graph else ex.run()
    runtime.sync()
    samples = []
    for _ in range(iters):
        t0 = time.perf_counter()
        ex.replay() if graph else ex.run()
        runtime.sync()
        samples.append((time.perf_counter() - t0) * 1e3)
    srt = sorted(samples)

    def rank(p):  # nearest rank, k = ceil(p * n), 1-indexed
        return srt[max(0, min(len(srt) - 1, int(np.ceil(p * len(srt))) - 1))]
    return {"latency_ms_mean": round(float(np.mean(samples)), 4), "latency_ms_p50": round(rank(0.50), 4),
            "latency_ms_p95": round(rank(0.95), 4), "iters": iters, "warmup": warmup}


class ClockSampler:
    """The GPU's shader (GFX) clock sampled every `period` seconds on a
    thread while the caller keeps the GPU busy, through amdsmi; of several
    visible GPUs, the one whose GFX activity was highest. None where amdsmi
    cannot read it (the reason is kept in `error`)."""

    def __init__(self, period: float = 0.01):
        self.period = period
        self.error = None
        self.handles = []
        self.samples = {}
        self._stop = None
        self._thread = None
        try:
            import amdsmi
            amdsmi.amdsmi_init()
            self.smi = amdsmi
            self.handles = list(amdsmi.amdsmi_get_processor_handles())
        except Exception as e:  # no driver access, no library
            self.error = f"amdsmi: {e}".splitlines()[0][:160]

    def _read(self, h):
        info = self.smi.amdsmi_get_clock_info(h, self.smi.AmdSmiClkType.GFX)
        act = self.smi.amdsmi_get_gpu_activity(h)
        return float(info["clk"]), float(act.get("gfx_activity", 0) if isinstance(act, dict) else 0)

    def _run(self):
        while not self._stop.is_set():
            for i, h in enumerate(self.handles):
                try:
                    self.samples.setdefault(i, []).append(self._read(h))
                except Exception as e:
                    self.error = f"amdsmi read: {e}".splitlines()[0][:160]
            self._stop.wait(self.period)

    def __enter__(self):
        import threading
        if self.handles:
            self._stop = threading.Event()
            self._thread = threading.Thread(target=self._run, daemon=True)
            self._thread.start()
        return self

    def __exit__(self, *exc):
        if self._thread:
            self._stop.set()
            self._thread.join(timeout=5)
        return False

    def result(self) -> dict | None:
        best = None
        for i, rows in self.samples.items():
            if not rows:
                continue
            clk = [r[0] for r in rows]
            act = float(np.mean([r[1] for r in rows]))
            # samples taken while the GPU reported itself busy: an idle
            # sample (the clock parked low between activity windows) says
            # nothing about the clock the kernels ran at
            busy = [r[0] for r in rows if r[1] >= 50.0]
            if best is None or act > best["gfx_activity_pct"]:
                best = {"mean_mhz": round(float(np.mean(clk)), 1),
                        "median_mhz": round(float(np.median(clk)), 1),
                        "busy_mean_mhz": round(float(np.mean(busy)), 1) if busy else None,
                        "busy_samples": len(busy),
                        "min_mhz": round(min(clk), 1), "max_mhz": round(max(clk), 1),
                        "samples": len(clk), "gfx_activity_pct": round(act, 1)}
        if best is None:
            return {"error": self.error or "no amdsmi samples"}
        best["source"] = ("amdsmi GFX clock and GFX activity, sampled every 10 ms during hipGraph "
                          "replays of the batch program; busy = samples with activity >= 50%")
        return best

    @staticmethod
    def kernel_mhz(clock: dict | None) -> float | None:
        """The clock the kernels ran at: the mean over busy samples where
        there are at least ten, else the median of all samples."""
        if not clock or "mean_mhz" not in clock:
            return None
        if clock.get("busy_samples", 0) >= 10 and clock.get("busy_mean_mhz"):
            return clock["busy_mean_mhz"]
        return clock["median_mhz"]


def kernel_table(ex, runtime, steps: int) -> list[dict]:
    """Per-kernel averages over `steps` directly launched nnc_run() calls
    (after one untimed call: the replays before it ran the same kernels from
    a graph)."""
    ex.run()
    runtime.sync()
    runtime.profile_reset()
    runtime.profile_enable(True)
    for _ in range(steps):
        ex.run()
    runtime.sync()
    table = runtime.profile_table()
    runtime.profile_enable(False)
    rows = []
    for r in table:
        avg_ms = r["ms"] / r["launches"]
        if r["flops"] > 0 and r["name"].startswith(MFMA_KERNELS):
            bound, unit, peak = "mfma", "TFLOP/s", PEAK_FP32_MFMA_TF
            achieved = r["flops"] / (r["ms"] * 1e-3) / 1e12
        elif r["name"].endswith("_fixup"):
            # stream-K partial-tile reduction: no algorithmic work of its own,
            # its time counts against the MFMA kernels it completes
            bound, unit, peak = "mfma-fixup", "TFLOP/s", PEAK_FP32_MFMA_TF
            achieved = 0.0
        else:
            bound, unit, peak = "hbm", "GB/s", PEAK_HBM_GBS
            achieved = r["bytes"] / (r["ms"] * 1e-3) / 1e9 if r["ms"] > 0 else 0.0
        rows.append({"kernel": r["name"], "launches_per_step": r["launches"] / steps,
                     "avg_us": round(avg_ms * 1e3, 2), "ms_per_step": round(r["ms"] / steps, 4),
                     "bound": bound, "achieved": round(achieved, 2), "unit": unit,
                     "frac": round(achieved / peak, 4),
                     "work_per_launch": (r["flops"] if bound == "mfma" else r["bytes"]) / r["launches"]})
    rows.sort(key=lambda x: -x["ms_per_step"])
    return rows


def _cpu_rate(lib, batch: int, warmup: int, iters: int) -> float:
    """Seconds per nnc_run() of the reference's own O3 call sequence for
    ResNet-18 at `batch` on a CPU implementation of the ABI (the mi355x
    target's fused and packed-weight entry points do not exist there)."""
    from nnc_py_amd.compiler import Executor, build_program, zoo
    prog = build_program(zoo.resnet18(batch=batch, seed=1), opt_level=3, target_passes=False)
    ex = Executor(prog, device=False, lib=lib)
    ex.set_input("input", np.random.default_rng(0).standard_normal((batch, 3, 224, 224)).astype(np.float32))
    for _ in range(warmup):
        ex.run()
    t0 = time.perf_counter()
    for _ in range(iters):
        ex.run()
    return (time.perf_counter() - t0) / iters


def cpu_baseline(pkg, iters_b1: int, iters_b32: int, batch: int) -> dict | None:
    """ResNet-18 through a CPU implementation of the same ABI, one thread:
    the reference runtime (runtime/x86/ops.c compiled by oracle/Makefile into
    oracle/_ref/) when present, else the oracle restatement. `value` at the
    benchmark's batch in the reference harness's quick mode (1 warmup + 3
    timed runs, benchmarks/harness.py:17-18), batch 1 beside it."""
    from nnc_py_amd import abi
    ref = ROOT / "oracle" / "_ref" / "libref_ops.so"
    port = ROOT / "oracle" / "liboracle.so"
    if ref.exists():
        path, kind = ref, "reference"
    elif port.exists():
        path, kind = port, "port"
    else:
        return None
    # the oracle's convolution uses OpenMP threads: pin it to one for a
    # one-thread figure (the reference's ops.c is single-threaded). libgomp
    # reads OMP_NUM_THREADS when it is loaded, so set it before the library
    # is, and also through omp_set_num_threads in case libgomp was loaded
    # earlier in this process
    os.environ["OMP_NUM_THREADS"] = "1"
    raw = ctypes.CDLL(str(path))
    try:
        raw.omp_set_num_threads(ctypes.c_int(1))
    except AttributeError:
        pass  # not an OpenMP build (the reference runtime)
    lib = abi.bind(raw)
    dt1 = _cpu_rate(lib, 1, 1, iters_b1)
    dtb = _cpu_rate(lib, batch, 1, iters_b32) if iters_b32 > 0 else None
    cpu = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    where = f"{path.relative_to(ROOT)} gcc -O2, 1 thread; host {cpu}, nproc {os.cpu_count()}"
    b1 = {"value": round(1.0 / dt1, 4), "unit": "images/s",
          "sample": f"batch 1: 1 warmup + {iters_b1} timed nnc_run() ({dt1:.2f} s each)"}
    if dtb is None:
        return {"value": b1["value"], "unit": "images/s", "cores": 1, "kind": kind,
                "sample": f"ResNet-18 fp32, the reference's O3 call sequence, {b1['sample']}, {where}"}
    return {"value": round(batch / dtb, 4), "unit": "images/s", "cores": 1, "kind": kind,
            "sample": (f"ResNet-18 fp32 batch {batch}, the reference's O3 call sequence, 1 warmup + {iters_b32} "
                       f"timed nnc_run() ({dtb:.2f} s each), {where}"),
            "b1": b1}


COPY_PROBE_BYTES = 256 << 20


def conv_symbol_pattern(name: str) -> re.Pattern | None:
    """Kernel-table name -> regex over the HIP kernel symbol rocprofv3 reports,
    e.g. conv_igemm_128x128_k3x3_v4 -> conv_streamk_k<nnc::Tile<128, 128, ...>, 3, 3, true>,
    conv_igemm_128x128_k3x3_dma -> conv_dma_k<nnc::Tile<128, 128, ...>, nnc::DmaPacked<..., 3, 3>, ...>."""
    m = re.fullmatch(r"conv_igemm_(\d+)x(\d+)_k(\d+)x(\d+)(c3)?_dma", name)
    if m:
        bm, bn, kh, kw, c3 = m.groups()
        loader = rf"DmaSmallC<nnc::Tile<[^>]*>, {kh}, {kw}, 3>" if c3 else rf"DmaPacked<nnc::Tile<[^>]*>, {kh}, {kw}>"
        return re.compile(rf"conv_dma_k<nnc::Tile<{bm}, {bn},[^>]*>, nnc::{loader}")
    m = re.fullmatch(r"conv_igemm_(\d+)x(\d+)_k(\d+|any)(?:x(\d+))?_(v4|s1)", name)
    if m:
        bm, bn, kh, kw, vec = m.groups()
        kh, kw = ("0", "0") if kh == "any" else (kh, kw)
        return re.compile(rf"conv_streamk_k<nnc::Tile<{bm}, {bn},[^>]*>, {kh}, {kw}, "
                          rf"{'true' if vec == 'v4' else 'false'}>")
    m = re.fullmatch(r"conv_stem_(rows|pool)_w(\d+)", name)
    if m:
        kernel = "conv_stem_k" if m.group(1) == "rows" else "conv_stem_pool_k"
        return re.compile(rf"{kernel}<{int(m.group(2)) // 16}>")
    m = re.fullmatch(r"gemm_mfma_(\d+)x(\d+)_\w+", name)
    if m:
        return re.compile(rf"gemm_streamk_k<nnc::Tile<{m.group(1)}, {m.group(2)},")
    m = re.fullmatch(r"gemm_dma_(\d+)x(\d+)_\w+", name)
    if m:
        return re.compile(rf"gemm_dma_k<nnc::Tile<{m.group(1)}, {m.group(2)},")
    return None


def pmc_child(args) -> int:
    """Run under rocprofv3 --pmc: two eager nnc_run() of the benchmark program,
    then a plain device copy of COPY_PROBE_BYTES (the calibration probe)."""
    load_package()
    from nnc_py_amd import runtime
    from nnc_py_amd.compiler import Executor, build_program, zoo
    lib = runtime.init(0)
    prog = build_program(zoo.resnet18(batch=args.batch, seed=1), opt_level=3)
    ex = Executor(prog, device=True)
    ex.set_input("input", np.random.default_rng(0).standard_normal((args.batch, 3, 224, 224)).astype(np.float32))
    for _ in range(2):
        ex.run()
    runtime.sync()
    ex.close()
    n = COPY_PROBE_BYTES // 4
    src = runtime.DeviceBuffer.empty((n,))
    dst = runtime.DeviceBuffer.empty((n,))
    ts, ks = src.tensor(), dst.tensor()
    for _ in range(3):
        lib.nnc_identity(ctypes.byref(ts[0]), ctypes.byref(ks[0]))
    runtime.sync()
    runtime.check(lib.nnc_hip_last_error(), "copy probe")
    return 0


def _pmc_run(counter: str, batch: int, timeout: int = 120) -> list[dict] | None:
    prof = shutil.which("rocprofv3")
    if not prof:
        return None
    with tempfile.TemporaryDirectory(prefix="nnc_pmc_") as tmp:
        cmd = ["timeout", "-s", "KILL", str(timeout), prof, "--pmc", counter, "--output-format", "csv",
               "-d", tmp, "-o", "pmc", "--", sys.executable, str(ROOT / "bench.py"), "--pmc-child",
               "--batch", str(batch)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        files = list(Path(tmp).rglob("*counter_collection.csv"))
        if res.returncode != 0 or not files:
            log(f"rocprofv3 --pmc {counter} failed (rc {res.returncode})")
            return None
        with open(files[0]) as f:
            return list(csv.DictReader(f))


def measure_traffic(kernel: str, batch: int) -> dict | None:
    """HBM bytes per launch of `kernel`: FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch, summed over channels), each scaled by COPY_PROBE_BYTES / the
    reading of the same counter for the copy probe's dispatches."""
    pat = conv_symbol_pattern(kernel)
    if pat is None:
        return None
    out = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        rows = _pmc_run(counter, batch)
        if not rows:
            return None
        per_dispatch: dict[tuple, float] = {}
        names: dict[tuple, str] = {}
        for r in rows:
            if r.get("Counter_Name") != counter:
                continue
            key = (r.get("Dispatch_Id"), r.get("Correlation_Id"))
            per_dispatch[key] = per_dispatch.get(key, 0.0) + float(r["Counter_Value"])
            names[key] = r.get("Kernel_Name", "")
        kern = [v for k, v in per_dispatch.items() if pat.search(names[k])]
        copy = [v for k, v in per_dispatch.items() if "copy16_k" in names[k]]
        if not kern or not copy:
            return None
        probe_kib = max(copy[-3:])  # the last dispatches are the 256 MiB probe copies
        scale = (COPY_PROBE_BYTES / 1024.0) / probe_kib
        out[counter] = {"kib_per_launch_raw": sum(kern) / len(kern), "probe_kib_raw": probe_kib,
                        "scale": scale, "bytes_per_launch": sum(kern) / len(kern) * 1024.0 * scale}
    return out


def _op_roofline(runtime, fn, reps: int = 10, warmup: int = 3) -> dict:
    """Per-kernel table of `fn()` (one or more nnc_* calls) over `reps` calls,
    each launch bracketed by its own hipEvent pair, and the same `reps` calls
    captured as one hipGraph and replayed back to back: `op_us` is the graph's
    time per call (no per-launch event overhead), `op_achieved` the call's
    algorithmic work over it."""
    for _ in range(warmup):
        fn()
    runtime.sync()
    runtime.profile_reset()
    runtime.profile_enable(True)
    for _ in range(reps):
        fn()
    runtime.sync()
    table = runtime.profile_table()
    runtime.profile_enable(False)
    rows = []
    flops = sum(r["flops"] for r in table) / reps
    nbytes = sum(r["bytes"] for r in table) / reps
    mfma = False
    for r in table:
        if r["flops"] > 0 and r["name"].startswith(MFMA_KERNELS):
            achieved, unit, peak = r["flops"] / (r["ms"] * 1e-3) / 1e12, "TFLOP/s", PEAK_FP32_MFMA_TF
            mfma = True
        else:
            achieved, unit, peak = (r["bytes"] / (r["ms"] * 1e-3) / 1e9 if r["ms"] > 0 else 0.0), "GB/s", PEAK_HBM_GBS
        rows.append({"kernel": r["name"], "launches": r["launches"] // reps, "avg_us": round(r["ms"] / r["launches"] * 1e3, 2),
                     "achieved": round(achieved, 2), "unit": unit, "frac": round(achieved / peak, 4)})
    lib = runtime.load()
    runtime.check(lib.nnc_hip_graph_begin(), "graph_begin")
    for _ in range(reps):
        fn()
    runtime.check(lib.nnc_hip_graph_end(), "graph_end")
    runtime.check(lib.nnc_hip_graph_launch(), "graph_launch")
    runtime.sync()
    launches = 5
    runtime.profile_reset()
    runtime.profile_enable(True)
    for _ in range(launches):
        runtime.check(lib.nnc_hip_graph_launch(), "graph_launch")
    runtime.sync()
    graph_ms = sum(r["ms"] for r in runtime.profile_table() if r["name"] == "graph")
    runtime.profile_enable(False)
    lib.nnc_hip_graph_destroy()
    op_us = graph_ms / (launches * reps) * 1e3
    if mfma:
        op_ach, unit, peak = flops / (op_us * 1e-6) / 1e12, "TFLOP/s", PEAK_FP32_MFMA_TF
    else:
        op_ach, unit, peak = nbytes / (op_us * 1e-6) / 1e9, "GB/s", PEAK_HBM_GBS
    return {"kernels": rows, "op_us": round(op_us, 2), "op_achieved": round(op_ach, 2), "op_unit": unit,
            "op_frac": round(op_ach / peak, 4)}


def _graph_us(runtime, fns, reps: int, launches: int = 5) -> float:
    """Microseconds per replay of one hipGraph holding `reps` rounds of the
    calls in `fns`."""
    lib = runtime.load()
    runtime.check(lib.nnc_hip_graph_begin(), "graph_begin")
    for _ in range(reps):
        for f in fns:
            f()
    runtime.check(lib.nnc_hip_graph_end(), "graph_end")
    runtime.check(lib.nnc_hip_graph_launch(), "graph_launch")
    runtime.sync()
    runtime.profile_reset()
    runtime.profile_enable(True)
    for _ in range(launches):
        runtime.check(lib.nnc_hip_graph_launch(), "graph_launch")
    runtime.sync()
    ms = sum(r["ms"] for r in runtime.profile_table() if r["name"] == "graph")
    runtime.profile_enable(False)
    lib.nnc_hip_graph_destroy()
    return ms / launches * 1e3


EVICT_BYTES = 320 << 20  # read by the eviction copy: more than the 256 MB Infinity Cache


def _cold_op_us(runtime, fn, reps: int = 10, rounds: int = 3) -> float:
    """Microseconds per call of `fn` with its inputs out of the Infinity
    Cache: a graph of `reps` x (a 320 MB device copy, then the call) less a
    graph of the copies alone, medians over `rounds` of each. Ops whose
    inputs fit the 256 MB cache otherwise read them back from it on every
    repeated call."""
    n = EVICT_BYTES // 4
    src = runtime.DeviceBuffer.empty((n,))
    dst = runtime.DeviceBuffer.empty((n,))
    ts, td = src.tensor(), dst.tensor()
    lib = runtime.load()

    def evict():
        lib.nnc_identity(ctypes.byref(ts[0]), ctypes.byref(td[0]))

    alone, both = [], []
    for _ in range(rounds):
        alone.append(_graph_us(runtime, [evict], reps))
        both.append(_graph_us(runtime, [evict, fn], reps))
    src.free()
    dst.free()
    return (float(np.median(both)) - float(np.median(alone))) / reps


def _copy_ceiling(runtime, nbytes: int, cold: bool = False) -> dict:
    """A plain device copy (copy16_k) that reads and writes `nbytes` each,
    timed like an op: the bandwidth a read-once/write-once kernel of this
    size reaches, ramp-up and tail included (and with `cold`, the same copy
    with its source out of the Infinity Cache, `_cold_op_us`)."""
    n = max(4, nbytes // 4)
    src = runtime.DeviceBuffer.empty((n,))
    dst = runtime.DeviceBuffer.empty((n,))
    ts, td = src.tensor(), dst.tensor()
    lib = runtime.load()
    fn = lambda: lib.nnc_identity(ctypes.byref(ts[0]), ctypes.byref(td[0]))  # noqa: E731
    res = _op_roofline(runtime, fn)
    out = {"bytes": 8 * n, "us": res["op_us"], "GB/s": res["op_achieved"], "frac": res["op_frac"]}
    if cold:
        cu = _cold_op_us(runtime, fn)
        out.update({"cold_us": round(cu, 2), "cold_frac": round(8 * n / (cu * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)})
    src.free()
    dst.free()
    return out


def run_suite() -> int:
    """The other workloads, one JSON line per item: GEMM sweep (Gemm
    M=N=K 1024/2048/4096 with bias, as emitted (transB=0) and after O3 weight
    packing (gemm_nt); batched MatMul [64,128,64]x[64,64,128]; vector MatMul
    [1,4096]x[4096,4096]), the bandwidth-bound ops at their workload sizes,
    and the 2-layer transformer encoder (B8 S128 D256 H4 FFN1024) as one
    hipGraph per step. Per-kernel achieved rates are algorithmic work over
    the library's per-launch hipEvent times."""
    load_package()
    from nnc_py_amd import abi, runtime
    from nnc_py_amd.compiler import Executor, build_program, zoo
    lib = runtime.init(0)
    rng = np.random.default_rng(0)
    keep = []

    def dev(arr, shape=None):
        """Device copy of `arr`; returns a Tensor* argument (kept alive in `keep`)."""
        buf = runtime.DeviceBuffer.from_array(np.ascontiguousarray(arr))
        t = buf.tensor(shape)
        keep.append((buf, t))
        return ctypes.pointer(t[0])

    def emit(suite, workload, res, copy_bytes=None, cold=None, **extra):
        """`cold`: the op's call again, timed with its inputs out of the
        Infinity Cache (`_cold_op_us`), for ops whose data fits it."""
        if cold:
            cu = _cold_op_us(runtime, cold)
            nbytes = res["op_achieved"] * 1e3 * res["op_us"]  # GB/s x us
            res["cold_op_us"] = round(cu, 2)
            res["cold_op_frac"] = round(nbytes / (cu * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)
        if copy_bytes:
            res["copy_ceiling"] = _copy_ceiling(runtime, copy_bytes, cold=bool(cold))
        print(json.dumps({"suite": suite, "workload": workload, **extra, **res}), flush=True)

    for n in (1024, 2048, 4096):
        a, b, c = (rng.uniform(-1, 1, s).astype(np.float32) for s in ((n, n), (n, n), (n,)))
        ta, tb, tc, to = dev(a), dev(b), dev(c), dev(np.zeros((n, n), np.float32))
        emit("gemm", f"Gemm {n}x{n}x{n} + bias[N], transB=0",
             _op_roofline(runtime, lambda: lib.nnc_gemm(ta, tb, tc, to, 1.0, 1.0, 0, 0)))
        tbt = dev(b.T.copy())
        emit("gemm", f"Gemm_nt {n}x{n}x{n} + bias[N] (O3 packed B)",
             _op_roofline(runtime, lambda: lib.nnc_gemm_nt(ta, tbt, tc, to, 1.0, 1.0)))
        keep.clear()
    ta, tb = dev(rng.uniform(-1, 1, (64, 128, 64)).astype(np.float32)), dev(rng.uniform(-1, 1, (64, 64, 128)).astype(np.float32))
    to = dev(np.zeros((64, 128, 128), np.float32))
    emit("gemm", "MatMul [64,128,64]x[64,64,128]", _op_roofline(runtime, lambda: lib.nnc_matmul(ta, tb, to)))
    tv, tm = dev(rng.uniform(-1, 1, (1, 4096)).astype(np.float32)), dev(rng.uniform(-1, 1, (4096, 4096)).astype(np.float32))
    to = dev(np.zeros((1, 4096), np.float32))
    emit("gemm", "MatMul [1,4096]x[4096,4096]", _op_roofline(runtime, lambda: lib.nnc_matmul(tv, tm, to)))
    keep.clear()

    shape = (32, 256, 56, 56)
    tx, ty = dev(rng.standard_normal(shape).astype(np.float32)), dev(rng.standard_normal(shape).astype(np.float32))
    to = dev(np.zeros(shape, np.float32))
    for op in ("nnc_add", "nnc_mul", "nnc_add_relu"):
        emit("bandwidth", f"{op} [32,256,56,56]", _op_roofline(runtime, lambda op=op: getattr(lib, op)(tx, ty, to)))
    for op in ("nnc_relu", "nnc_sigmoid", "nnc_tanh"):
        emit("bandwidth", f"{op} [32,256,56,56]", _op_roofline(runtime, lambda op=op: getattr(lib, op)(tx, to)),
             copy_bytes=4 * 32 * 256 * 56 * 56 if op == "nnc_relu" else None)
    emit("bandwidth", "nnc_clip(-6,6) [32,256,56,56]", _op_roofline(runtime, lambda: lib.nnc_clip(tx, to, -6.0, 6.0)))
    tcat = dev(np.zeros((32, 512, 56, 56), np.float32))
    pair = (abi.TP * 2)(tx, ty)
    emit("bandwidth", "nnc_concat axis 1: 2 x [32,256,56,56]",
         _op_roofline(runtime, lambda: lib.nnc_concat(ctypes.cast(pair, abi.TPP), tcat, 2, 1)),
         copy_bytes=4 * 32 * 512 * 56 * 56)
    emit("bandwidth", "nnc_split axis 1: [32,512,56,56] -> 2",
         _op_roofline(runtime, lambda: lib.nnc_split(tcat, ctypes.cast(pair, abi.TPP), 2, 1)))
    keep.clear()
    ts, tso = dev(rng.standard_normal((4096, 1024)).astype(np.float32)), dev(np.zeros((4096, 1024), np.float32))
    sm = lambda: lib.nnc_softmax(ts, tso, -1)  # noqa: E731
    emit("bandwidth", "nnc_softmax [4096,1024] axis -1", _op_roofline(runtime, sm), copy_bytes=4 * 4096 * 1024, cold=sm)
    tl, tg, tb0 = dev(rng.standard_normal((8192, 768)).astype(np.float32)), dev(np.ones(768, np.float32)), dev(np.zeros(768, np.float32))
    tlo = dev(np.zeros((8192, 768), np.float32))
    ln = lambda: lib.nnc_layernorm(tl, tg, tb0, tlo, -1, 1e-5)  # noqa: E731
    emit("bandwidth", "nnc_layernorm [8192,768] eps 1e-5", _op_roofline(runtime, ln), copy_bytes=4 * 8192 * 768, cold=ln)
    r = rng.standard_normal((32, 512, 28, 28)).astype(np.float32)
    tr, tro = dev(r, (32, 512, 784)), dev(np.zeros((32, 512, 1), np.float32))
    for op in ("nnc_reducemean", "nnc_reducesum"):
        rd = lambda op=op: getattr(lib, op)(tr, tro, 2, 1)  # noqa: E731
        emit("bandwidth", f"{op} axes (2,3) of [32,512,28,28]", _op_roofline(runtime, rd), cold=rd)
    keep.clear()

    # the element-wise chain relu(x + y) * x, clip(-6, 6), sigmoid, + t as one
    # nnc_hip_fused_eltwise pass (three inputs read, one output written)
    tx, ty, tt = (dev(rng.standard_normal(shape).astype(np.float32)) for _ in range(3))
    to = dev(np.zeros(shape, np.float32))
    ins3 = (abi.TP * 3)(tx, ty, tt)
    prog5 = (ctypes.c_int * 15)(4, 0, 1, 2, -1, 0, 9, -1, -1, 7, -1, -1, 0, -1, 2)
    consts5 = (ctypes.c_float * 10)(0, 0, 0, 0, -6, 6, 0, 0, 0, 0)
    emit("bandwidth", "nnc_hip_fused_eltwise: relu(x+y)*x, clip, sigmoid, +t [32,256,56,56]",
         _op_roofline(runtime, lambda: lib.nnc_hip_fused_eltwise(ctypes.cast(ins3, abi.TPP), 3, prog5, 5, consts5, to)))
    keep.clear()
    # the whole chain program (config's element-wise chain, softmax, layernorm
    # and reductions) at O3 on this target, and the reference's own O3 call
    # sequence on this library, one hipGraph per step
    for label, target in (("mi355x O3 (fused element-wise chains, no Concat -> Split)", True),
                          ("reference O3 call sequence", False)):
        prog = build_program(zoo.bandwidth_chain(seed=1), opt_level=3, target_passes=target)
        ex = Executor(prog, device=True)
        for k in ("x", "y", "s", "l", "r"):
            ex.set_input(k, rng.standard_normal(prog.graph.tensors[k].shape).astype(np.float32))
        steps = 20
        dt = timed_steps(ex, steps, 5, True, runtime)
        emit("bandwidth", f"bandwidth chain program, {label}, hipGraph", {"kernels": kernel_table(ex, runtime, 3)},
             ms_per_step=round(dt / steps * 1e3, 4), calls=len(prog.calls))
        ex.close()

    prog = build_program(zoo.transformer_encoder(seed=1), opt_level=3)
    ex = Executor(prog, device=True)
    ex.set_input("input", (rng.standard_normal((8, 128, 256)) * 0.02).astype(np.float32))
    steps = 50
    dt = timed_steps(ex, steps, 10, True, runtime)
    ms = dt / steps * 1e3
    flops = zoo.transformer_flops()
    emit("transformer", "encoder 2 layers, B8 S128 D256 H4 FFN1024, O3, hipGraph", {"kernels": kernel_table(ex, runtime, 5)},
         ms_per_step=round(ms, 4), gflops_per_s=round(flops / (ms * 1e-3) / 1e9, 1),
         mfma_frac_whole_step=round(flops / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TF, 4))
    ex.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--no-graph", action="store_true", help="launch each nnc_* call instead of a hipGraph")
    ap.add_argument("--profile-steps", type=int, default=20)
    ap.add_argument("--latency-batches", default="1,8,16,32",
                    help="batches timed per step as the reference harness does (mean/p50/p95; '' skips)")
    ap.add_argument("--clock-seconds", type=float, default=1.0,
                    help="seconds of graph replays at the benchmark batch while the shader clock is sampled (0 skips)")
    ap.add_argument("--cpu-iters", type=int, default=10, help="timed batch-1 runs of the CPU baseline")
    ap.add_argument("--cpu-iters-batch", type=int, default=3,
                    help="timed runs of the CPU baseline at the benchmark batch (0: batch 1 only)")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--no-b1", action="store_true", help="measure batch 32 only (profiling runs)")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 --pmc traffic runs")
    ap.add_argument("--no-dropin", action="store_true",
                    help="skip the reference's own O3 call sequence on the HIP library")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--suite", action="store_true",
                    help="instead of the ResNet-18 line: GEMM sweep, bandwidth ops and transformer encoder, "
                         "one JSON line each")
    args = ap.parse_args()
    if args.pmc_child:
        return pmc_child(args)
    if args.suite:
        if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
            print("bench.py --suite measures one GPU", file=sys.stderr)
            return 2
        return run_suite()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the nnc program runs on a single MI355X "
              f"(--gpus {args.gpus}, WORLD_SIZE {world} requested); multi-GPU batch sharding is "
              f"not launched.", file=sys.stderr)
        return 2

    pkg = load_package()
    from nnc_py_amd import runtime
    from nnc_py_amd.compiler import Executor, build_program, zoo
    runtime.init(0)
    graph = not args.no_graph
    results = {}
    tables = {}
    clock = None
    lat_batches = [int(b) for b in args.latency_batches.split(",") if b.strip()]
    runs = [(args.batch, args.steps)] + ([] if args.no_b1 else [(1, max(args.steps, 50))])
    runs += [(b, 20) for b in lat_batches if b not in dict(runs)]
    for batch, steps in runs:
        log(f"building ResNet-18 batch {batch}")
        prog = build_program(zoo.resnet18(batch=batch, seed=1), opt_level=3)
        ex = Executor(prog, device=True)
        x = np.random.default_rng(0).standard_normal((batch, 3, 224, 224)).astype(np.float32)
        ex.set_input("input", x)
        log(f"batch {batch}: {args.warmup} warmup + {steps} timed steps (graph={graph})")
        dt = timed_steps(ex, steps, args.warmup, graph, runtime)
        out = ex.get("output")
        if not np.isfinite(out).all():
            log("non-finite output")
            return 1
        results[batch] = {"images_per_s": batch * steps / dt, "ms_per_step": dt / steps * 1e3, "steps": steps}
        log(f"batch {batch}: {results[batch]['ms_per_step']:.3f} ms/step, "
            f"{results[batch]['images_per_s']:.1f} images/s")
        if batch in lat_batches:
            results[batch]["latency"] = latency_samples(ex, 20, 5, graph, runtime)
            log(f"batch {batch}: per-step latency p50 {results[batch]['latency']['latency_ms_p50']:.3f} ms, "
                f"p95 {results[batch]['latency']['latency_ms_p95']:.3f} ms")
        if batch == args.batch and args.clock_seconds > 0 and graph:
            sampler = ClockSampler()
            with sampler:
                t_end = time.perf_counter() + args.clock_seconds
                while time.perf_counter() < t_end:
                    for _ in range(10):
                        ex.replay()
                    runtime.sync()
            clock = sampler.result()
            log(f"shader clock during replays: {clock}")
        if batch == args.batch:
            tables[batch] = kernel_table(ex, runtime, args.profile_steps)
        ex.close()

    # the drop-in path: the call sequence the reference's own O3 pipeline
    # emits (reference entry points only) on this library, same batch
    dropin = None
    if not args.no_dropin:
        prog = build_program(zoo.resnet18(batch=args.batch, seed=1), opt_level=3, target_passes=False)
        ex = Executor(prog, device=True)
        ex.set_input("input", np.random.default_rng(0).standard_normal((args.batch, 3, 224, 224)).astype(np.float32))
        steps = max(10, args.steps // 2)
        log(f"drop-in (reference O3 call sequence, {len(prog.calls)} calls): {steps} timed steps")
        dt = timed_steps(ex, steps, args.warmup, graph, runtime)
        dropin = {"images_per_s": round(args.batch * steps / dt, 2), "ms_per_step": round(dt / steps * 1e3, 4),
                  "calls": len(prog.calls), "batch": args.batch}
        ex.close()

    table = tables[args.batch]
    dom = table[0]
    peak = PEAK_FP32_MFMA_TF if dom["bound"] == "mfma" else PEAK_HBM_GBS
    traffic = None
    traffic_detail = None
    if not args.no_traffic:
        log(f"HBM traffic of {dom['kernel']}: rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE")
        traffic_detail = measure_traffic(dom["kernel"], args.batch)
        if traffic_detail:
            traffic = round(traffic_detail["FETCH_SIZE"]["bytes_per_launch"]
                            + traffic_detail["WRITE_SIZE"]["bytes_per_launch"])
    roofline = {"kernel": dom["kernel"], "bound": dom["bound"], "achieved": dom["achieved"],
                "peak": peak, "unit": dom["unit"], "frac": round(dom["achieved"] / peak, 4),
                "traffic": traffic, "avg_launch_us": dom["avg_us"],
                "work_per_launch": dom["work_per_launch"]}
    mhz = ClockSampler.kernel_mhz(clock)
    if mhz:
        # the published peak assumes the 2.4 GHz peak engine clock; the
        # kernel ran at the sampled clock
        roofline["shader_clock_mhz"] = mhz
        roofline["frac_at_clock"] = round(dom["achieved"] / (peak * mhz / 2400.0), 4)
    if traffic_detail:
        roofline["traffic_detail"] = {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in traffic_detail.items()}
    gpu_ms = sum(r["ms_per_step"] for r in table)
    conv_ms = sum(r["ms_per_step"] for r in table if r["bound"] in ("mfma", "mfma-fixup"))
    conv_flops = zoo.resnet18_flops(args.batch)

    cpu = None
    if not args.skip_cpu:
        log(f"CPU baseline: ResNet-18 batch 1 ({args.cpu_iters} timed runs) and batch {args.batch} "
            f"({args.cpu_iters_batch} timed runs), one thread")
        cpu = cpu_baseline(pkg, args.cpu_iters, args.cpu_iters_batch, args.batch)

    b = results[args.batch]
    line = {
        "metric": METRIC,
        "value": round(b["images_per_s"], 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": b["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(b["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: x ~ N(0,1) seed 0; He-normal conv/FC weights, biases N(0, 0.01^2), seed 1",
        "config": {"workload": "ResNet-18 fp32 (BN folded), batch 32, 3x224x224, O3 nnc program, one hipGraph per step",
                   "batch": args.batch, "opt_level": 3, "graph": graph},
        "b1": ({"images_per_s": round(results[1]["images_per_s"], 2),
                "ms_per_step": round(results[1]["ms_per_step"], 4)} if 1 in results else None),
        "roofline": roofline,
        "mfma_frac_all_conv": round(conv_flops / (conv_ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TF, 4) if conv_ms else None,
        "kernel_ms_per_step": round(gpu_ms, 4),
        "per_kernel": [{k: r[k] for k in ("kernel", "launches_per_step", "avg_us", "bound", "achieved", "unit", "frac")}
                       for r in table],
        "per_kernel_timing": ("hipEvent pair on the library stream around each launch of directly launched nnc_run() "
                              "calls: a launch of a few microseconds reads about 2.5 us long (event overhead), so "
                              "small kernels' frac is understated; rocprofv3 kernel durations are in profiles/"),
        "batches": {str(bt): {"images_per_s": round(r["images_per_s"], 2), "ms_per_step": round(r["ms_per_step"], 4),
                              **r.get("latency", {})} for bt, r in sorted(results.items())},
        "shader_clock": clock,
        "cpu_baseline": cpu,
        "dropin": dropin,
        "host": platform.node(),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
