"""nnc_hip_conv_packed_noalloc, the allocation-free variant of
nnc_hip_conv_packed (stream-K partials and tile counters in a static device
array instead of the grow-only workspace).

Two calls in a row through the C-ABI - a ResNet-18 batch-32 layer-2 shape
(128x128 tiles, stream-K with a fixup launch) and then a smaller batch-2
64-channel shape (64x128 tiles whose shared tiles are finished in-kernel
through the static tile counters) - each equal bit for bit to
nnc_hip_conv_packed on the same inputs (same kernels, same stream-K plan)
and within 1e-4 abs / 1e-3 rel of the oracle. A thread without library state
gets NNC_HIP_ESTATE and no launch: the entry point never creates it.
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
    (2, 64, 56, 64, 3, 1, 1),     # smaller: 64x128 tiles, in-kernel finish on the counters
]


def test_noalloc_matches_conv_packed_twice(hip, dmem, abi, oracle_lib):
    from nnc_py_amd import runtime
    for i, shape in enumerate(SHAPES):
        case = _packed_case(np.random.default_rng(20 + i), *shape, act=1, bias=True, res=i == 0)
        print(f"no-alloc call {i}: {case['name']}", flush=True)
        want = caserun.run_case(hip, case, abi, dmem)["out"]
        assert runtime.last_error()[0] == 0, runtime.last_error()[1]
        fixed = dict(case, op="nnc_hip_conv_packed_noalloc")
        got = caserun.run_case(hip, fixed, abi, dmem)["out"]
        assert runtime.last_error()[0] == 0, runtime.last_error()[1]
        assert caserun.same_bits(got, want), f"{case['name']}: differs from nnc_hip_conv_packed"
        exp = caserun.run_case(oracle_lib, case, abi)["out"]
        bad = caserun.fp_violations(got, exp, 1e-4, 1e-3)
        assert bad.size == 0, f"{case['name']}: {bad.size} outputs outside the bar"
        dmem.release()


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
