"""Generic driver for one nnc_* call described as data.

A case is a dict:
    name     unique id
    op       nnc_* entry point
    tensors  {key: numpy array}  inputs and the initial contents of outputs
    args     call arguments in order, each one of
               ("t", key)          Tensor* bound to tensors[key]
               ("null",)           NULL Tensor*
               ("i", int) / ("f", float)
               ("tl", [keys])      Tensor** array
               ("i64", [ints])     int64_t* array
               ("i64null",)        NULL int64_t*
               ("i32", [ints])     int* array
               ("f32", [floats])   float* array
    outputs  keys whose contents are compared after the call
    bar      "exact" (bit-for-bit, NaN == NaN) or "fp" (atol/rtol rule)

The same case runs against the reference runtime (host memory), the oracle
(host memory) and libnnc_hip.so (device memory via a `mem` adapter).
"""

from __future__ import annotations

import ctypes

import numpy as np


class HostMem:
    """Tensors live in numpy arrays; pointers are host addresses."""

    def __init__(self):
        self.keep = []

    def place(self, arr: np.ndarray) -> int:
        a = np.ascontiguousarray(arr).copy()
        self.keep.append(a)
        return a.ctypes.data, a

    def fetch(self, handle, arr_like: np.ndarray) -> np.ndarray:
        return handle.copy()

    def finish(self):
        pass


def build_call(case: dict, abi, mem):
    """Materialise the case's arguments; returns (args, handles, keepalive)."""
    keep = []
    handles = {}
    tensors = {}
    for key, arr in case["tensors"].items():
        ptr, handle = mem.place(arr)
        handles[key] = handle
        dtype = abi.NUMPY_TO_NNC[arr.dtype.name]
        t, sh = abi.make_tensor(ptr, dtype, arr.shape, arr.nbytes)
        keep.append(sh)
        tensors[key] = t
    args = []
    for spec in case["args"]:
        kind = spec[0]
        if kind == "t":
            args.append(ctypes.pointer(tensors[spec[1]]))
        elif kind == "null":
            args.append(None)
        elif kind == "i":
            args.append(int(spec[1]))
        elif kind == "f":
            args.append(float(spec[1]))
        elif kind == "tl":
            arr = (abi.TP * len(spec[1]))(*[ctypes.pointer(tensors[k]) for k in spec[1]])
            keep.append(arr)
            args.append(ctypes.cast(arr, abi.TPP))
        elif kind == "i64":
            arr = (ctypes.c_int64 * max(1, len(spec[1])))(*[int(v) for v in spec[1]])
            keep.append(arr)
            args.append(ctypes.cast(arr, abi.I64P))
        elif kind == "i64null":
            args.append(None)
        elif kind == "i32":
            arr = (ctypes.c_int * max(1, len(spec[1])))(*[int(v) for v in spec[1]])
            keep.append(arr)
            args.append(ctypes.cast(arr, abi.I32P))
        elif kind == "f32":
            arr = (ctypes.c_float * max(1, len(spec[1])))(*[float(v) for v in spec[1]])
            keep.append(arr)
            args.append(ctypes.cast(arr, abi.F32P))
        else:
            raise ValueError(f"unknown arg kind {kind!r}")
    return args, handles, (keep, tensors)


def run_case(lib, case: dict, abi, mem=None) -> dict:
    """Call case['op'] on `lib`; return {output key: resulting array}."""
    mem = mem or HostMem()
    args, handles, keep = build_call(case, abi, mem)
    getattr(lib, case["op"])(*args)
    mem.finish()
    out = {}
    for key in case["outputs"]:
        like = case["tensors"][key]
        out[key] = np.asarray(mem.fetch(handles[key], like)).reshape(like.shape)
    del keep
    return out


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit-for-bit equality (NaN payloads included)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and a.tobytes() == b.tobytes()


def fp_violations(got: np.ndarray, ref: np.ndarray, atol=1e-4, rtol=1e-3) -> np.ndarray:
    """Indices failing the reference pass rule diff <= atol or diff <= rtol*|ref|
    (tests/test_common.py:439 of the reference); NaN must match NaN."""
    g = got.astype(np.float64).ravel()
    r = ref.astype(np.float64).ravel()
    nan_g, nan_r = np.isnan(g), np.isnan(r)
    both = nan_g & nan_r
    with np.errstate(invalid="ignore"):
        diff = np.abs(g - r)
        ok = (diff <= atol) | (diff <= rtol * np.abs(r)) | both | (g == r)
    return np.nonzero(~ok)[0]
