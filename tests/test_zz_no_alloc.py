"""nnc_hip_conv_packed_noalloc, the allocation-free variant of
nnc_hip_conv_packed (stream-K partials and tile counters in a static device
array instead of the grow-only workspace).

Three calls in a row through the C-ABI, each on a smaller input than the
last - a ResNet-18 batch-32 layer-2 shape (128x128 tiles, stream-K with a
fixup launch), a 12-image 64-channel shape (64x128 tiles whose shared tiles
are finished in-kernel through the static tile counters) and a batch-1
512-channel 7x7 shape (short-convolution tiles split over 8 workgroups,
finished through the static counters too) - each equal bit for bit to
nnc_hip_conv_packed on the same inputs (same kernels, same plans) and within
1e-4 abs / 1e-3 rel of the oracle. A thread without library state
gets NNC_HIP_ESTATE and no launch: the entry point never creates it. Calls
from two host threads on their own streams are ordered on the device, so
they do not race on the shared array.
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np
import pytest

import caserun
from test_hip_kernels import _packed_case

pytestmark = pytest.mark.gpu

SHAPES = [
    (32, 128, 28, 128, 3, 1, 1),  # 128x128 tiles, stream-K with the fixup kernel
    (12, 64, 56, 64, 3, 1, 1),    # smaller: 64x128 tiles, in-kernel finish on the counters
    (1, 512, 7, 512, 3, 1, 1),    # smaller still: short-convolution tiles split 8 ways, on the counters
]


def test_noalloc_matches_conv_packed_twice(hip, dmem, abi, oracle_lib):
    from nnc_py_amd import runtime
    for i, shape in enumerate(SHAPES):
        case = _packed_case(np.random.default_rng(20 + i), *shape, act=1, bias=True, res=i != 2)
        print(f"no-alloc call {i}: {case['name']}", flush=True)
        runtime.profile_reset()
        runtime.profile_enable(True)
        want = caserun.run_case(hip, case, abi, dmem)["out"]
        launched = {r["name"] for r in runtime.profile_table()}
        runtime.profile_enable(False)
        assert runtime.last_error()[0] == 0, runtime.last_error()[1]
        # the plan both entry points share: the first shape's tiles finished
        # by the fixup kernel, the others' in their kernels on the counters
        # (the no-alloc calls record no launch table)
        assert any("fixup" in n for n in launched) == (i == 0), sorted(launched)
        fixed = dict(case, op="nnc_hip_conv_packed_noalloc")
        got = caserun.run_case(hip, fixed, abi, dmem)["out"]
        assert runtime.last_error()[0] == 0, runtime.last_error()[1]
        assert caserun.same_bits(got, want), f"{case['name']}: differs from nnc_hip_conv_packed"
        exp = caserun.run_case(oracle_lib, case, abi)["out"]
        bad = caserun.fp_violations(got, exp, 1e-4, 1e-3)
        assert bad.size == 0, f"{case['name']}: {bad.size} outputs outside the bar"
        dmem.release()


def test_noalloc_calls_from_two_threads_are_ordered(hip, abi, oracle_lib):
    """Two host threads, each on its own library stream, start together and
    alternate no-alloc calls on the batch-32 shape (its stream-K partials
    and fixup in the shared static array) with their own inputs and
    outputs, four calls each without synchronising in between: every call
    waits on the device for the previous one, so each thread's output
    equals its nnc_hip_conv_packed result bit for bit."""
    from nnc_py_amd import runtime
    cases = [_packed_case(np.random.default_rng(40 + i), *SHAPES[0], act=1, bias=True, res=False) for i in range(2)]
    results, errors = {}, []
    start = threading.Barrier(2)

    def worker(i):
        try:
            case = cases[i]
            bufs = {k: runtime.DeviceBuffer.from_array(np.ascontiguousarray(v)) for k, v in case["tensors"].items()}
            ts = {k: b.tensor() for k, b in bufs.items()}
            args = [ctypes.byref(ts[a[1]][0]) if a[0] == "t" else (None if a[0] == "null" else a[1])
                    for a in case["args"]]
            hip.nnc_hip_conv_packed(*args)  # creates this thread's library state
            runtime.sync()
            want = bufs["out"].to_array()
            start.wait(timeout=60)
            for _ in range(4):
                hip.nnc_hip_conv_packed_noalloc(*args)
            runtime.sync()
            results[i] = (bufs["out"].to_array(), want)
            for b in bufs.values():
                b.free()
        except Exception as e:  # reported by the main thread
            errors.append(f"thread {i}: {e!r}")

    print("no-alloc: two threads, four calls each", flush=True)
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    assert runtime.last_error()[0] == 0, runtime.last_error()[1]
    for i in range(2):
        got, want = results[i]
        assert caserun.same_bits(got, want), f"thread {i}: no-alloc output differs from nnc_hip_conv_packed"
        exp = caserun.run_case(oracle_lib, cases[i], abi)["out"]
        assert caserun.fp_violations(got, exp, 1e-4, 1e-3).size == 0


def test_noalloc_needs_the_threads_library_state(hip, abi):
    """A fresh thread's first call is the no-alloc entry point: it fails
    with NNC_HIP_ESTATE instead of creating the thread's streams and scratch
    (which would allocate)."""
    from nnc_py_amd import runtime
    runtime.clear_error()
    out = {}

    def fresh():
        null = ctypes.POINTER(abi.Tensor)()
        hip.nnc_hip_conv_packed_noalloc(null, null, null, null, null, 3, 3, 1, 1, 1, 1, 1)
        out["code"] = runtime.last_error()[0]

    t = threading.Thread(target=fresh)
    t.start()
    t.join(timeout=60)
    assert out.get("code") == 5  # NNC_HIP_ESTATE
    runtime.clear_error()
