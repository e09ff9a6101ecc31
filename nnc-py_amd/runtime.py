"""Host-side binding of libnnc_hip.so (include/nnc_hip.h + include/nnc_ops.h).

    from nnc_py_amd import runtime
    lib = runtime.load()          # raises if lib/libnnc_hip.so was not built
    runtime.init(0)
    buf = runtime.DeviceBuffer.from_array(x)   # hipMalloc + upload
    ...
    runtime.sync(); y = buf.to_array()

There is no CPU fallback: every nnc_* call goes to the gfx950 kernels.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

from . import abi

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libnnc_hip.so"

_lib = None

_HIP_SIGNATURES = {
    "nnc_hip_init": ([ctypes.c_int], ctypes.c_int),
    "nnc_hip_shutdown": ([], None),
    "nnc_hip_arena_reserve": ([ctypes.c_size_t], ctypes.c_int),
    "nnc_hip_arena_base": ([], ctypes.c_void_p),
    "nnc_hip_arena_size": ([], ctypes.c_size_t),
    "nnc_hip_bind": ([abi.TP, ctypes.c_size_t], ctypes.c_int),
    "nnc_hip_spill_reserve": ([ctypes.c_size_t], ctypes.c_int),
    "nnc_hip_spill_base": ([], ctypes.c_void_p),
    "nnc_hip_bind_spill": ([abi.TP, ctypes.c_size_t], ctypes.c_int),
    "nnc_hip_malloc": ([ctypes.c_size_t], ctypes.c_void_p),
    "nnc_hip_free": ([ctypes.c_void_p], None),
    "nnc_hip_host_malloc": ([ctypes.c_size_t], ctypes.c_void_p),
    "nnc_hip_host_free": ([ctypes.c_void_p], None),
    "nnc_hip_upload": ([abi.TP, ctypes.c_void_p], ctypes.c_int),
    "nnc_hip_download": ([abi.TP, ctypes.c_void_p], ctypes.c_int),
    "nnc_hip_memcpy_h2d": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int),
    "nnc_hip_memcpy_d2h": ([ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int),
    "nnc_hip_sync": ([], ctypes.c_int),
    "nnc_hip_stream": ([], ctypes.c_void_p),
    "nnc_hip_last_error": ([], ctypes.c_int),
    "nnc_hip_last_error_message": ([], ctypes.c_char_p),
    "nnc_hip_clear_error": ([], None),
    "nnc_hip_profile_enable": ([ctypes.c_int], None),
    "nnc_hip_profile_reset": ([], None),
    "nnc_hip_profile_count": ([], ctypes.c_int),
    "nnc_hip_profile_entry": ([ctypes.c_int, ctypes.c_char_p, ctypes.c_int,
                               ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_double)],
                              ctypes.c_int),
    "nnc_hip_profile_work": ([ctypes.c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)],
                             ctypes.c_int),
    "nnc_hip_debug_dump": ([abi.TP, ctypes.c_char_p, ctypes.c_int, ctypes.c_void_p], ctypes.c_int),
    "nnc_hip_stream_fork": ([], ctypes.c_int),
    "nnc_hip_stream_select": ([ctypes.c_int], ctypes.c_int),
    "nnc_hip_stream_join": ([], ctypes.c_int),
    "nnc_hip_graph_begin": ([], ctypes.c_int),
    "nnc_hip_graph_end": ([], ctypes.c_int),
    "nnc_hip_graph_launch": ([], ctypes.c_int),
    "nnc_hip_graph_destroy": ([], None),
    "nnc_hip_conv_add_relu": (abi.TARGET_SIGNATURES["nnc_hip_conv_add_relu"], None),
    "nnc_hip_conv_packed": (abi.TARGET_SIGNATURES["nnc_hip_conv_packed"], None),
    "nnc_hip_transfer": (abi.TARGET_SIGNATURES["nnc_hip_transfer"], None),
    "nnc_hip_conv_proj": (abi.TARGET_SIGNATURES["nnc_hip_conv_proj"], None),
    "nnc_hip_conv_packed_noalloc": (abi.TARGET_SIGNATURES["nnc_hip_conv_packed_noalloc"], None),
    "nnc_hip_gap_gemm_nt": (abi.TARGET_SIGNATURES["nnc_hip_gap_gemm_nt"], None),
    "nnc_hip_conv_maxpool": (abi.TARGET_SIGNATURES["nnc_hip_conv_maxpool"], None),
    "nnc_hip_fused_eltwise": (abi.TARGET_SIGNATURES["nnc_hip_fused_eltwise"], None),
    "nnc_hip_add_layernorm": (abi.TARGET_SIGNATURES["nnc_hip_add_layernorm"], None),
    "nnc_hip_scaled_softmax": (abi.TARGET_SIGNATURES["nnc_hip_scaled_softmax"], None),
    "nnc_hip_transpose_slice": (abi.TARGET_SIGNATURES["nnc_hip_transpose_slice"], None),
    "nnc_hip_attention": (abi.TARGET_SIGNATURES["nnc_hip_attention"], None),
    "nnc_hip_ew_chain_specialized": ([ctypes.c_int, abi.I32P, ctypes.c_int], ctypes.c_int),
}


class HipError(RuntimeError):
    pass


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and bind libnnc_hip.so (`path`, else $NNC_HIP_LIB, else
    the in-tree build). Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path or os.environ.get("NNC_HIP_LIB") or LIB_PATH)
    if not p.exists():
        raise HipError(f"{p} is not built; run `python nnc-py_amd/build.py` (or __graft_entry__.build())")
    # RTLD_LOCAL: the library's nnc_* names must not interpose on another
    # implementation of the ABI loaded in the same process (the CPU oracle)
    lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_LOCAL)
    abi.bind(lib)
    for name, (args, res) in _HIP_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def check(code: int, what: str = "") -> None:
    if code != 0:
        msg = _lib.nnc_hip_last_error_message().decode(errors="replace") if _lib else ""
        raise HipError(f"{what} failed with code {code}: {msg}")


def init(device: int = 0) -> ctypes.CDLL:
    lib = load()
    check(lib.nnc_hip_init(device), "nnc_hip_init")
    return lib


def sync() -> None:
    check(load().nnc_hip_sync(), "nnc_hip_sync")


def last_error() -> tuple[int, str]:
    lib = load()
    return lib.nnc_hip_last_error(), lib.nnc_hip_last_error_message().decode(errors="replace")


def clear_error() -> None:
    load().nnc_hip_clear_error()


class DeviceBuffer:
    """One hipMalloc'd allocation holding a numpy-shaped array."""

    def __init__(self, nbytes: int, shape, dtype):
        self.lib = load()
        self.nbytes = int(nbytes)
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.ptr = self.lib.nnc_hip_malloc(max(16, self.nbytes))
        if not self.ptr:
            raise HipError(f"nnc_hip_malloc({self.nbytes}) failed: {last_error()[1]}")

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        buf = cls(a.nbytes, a.shape, a.dtype)
        if a.nbytes:
            check(buf.lib.nnc_hip_memcpy_h2d(buf.ptr, a.ctypes.data, a.nbytes), "upload")
        return buf

    @classmethod
    def empty(cls, shape, dtype=np.float32) -> "DeviceBuffer":
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return cls(n, shape, dtype)

    def to_array(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(self.lib.nnc_hip_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes), "download")
        return out

    def upload(self, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        check(self.lib.nnc_hip_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes), "upload")

    def tensor(self, shape=None):
        """(Tensor, keepalive) describing this buffer (optionally reshaped)."""
        shape = self.shape if shape is None else tuple(shape)
        return abi.make_tensor(self.ptr, abi.NUMPY_TO_NNC[self.dtype.name], shape, self.nbytes)

    def free(self) -> None:
        if self.ptr:
            self.lib.nnc_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceMem:
    """Memory adapter for the case runner: tensors live in device buffers."""

    def __init__(self):
        self.bufs = []

    def place(self, arr: np.ndarray):
        buf = DeviceBuffer.from_array(arr)
        self.bufs.append(buf)
        return buf.ptr, buf

    def fetch(self, handle, arr_like):
        return handle.to_array()

    def finish(self):
        sync()

    def release(self):
        for b in self.bufs:
            b.free()
        self.bufs.clear()


def profile_enable(on: bool = True) -> None:
    load().nnc_hip_profile_enable(1 if on else 0)


def profile_reset() -> None:
    load().nnc_hip_profile_reset()


def profile_table() -> list[dict]:
    """Per kernel name since the last reset: launches, total ms, and the
    algorithmic flops / bytes of those launches."""
    lib = load()
    out = []
    name = ctypes.create_string_buffer(128)
    for i in range(lib.nnc_hip_profile_count()):
        launches = ctypes.c_int64()
        ms = ctypes.c_double()
        flops = ctypes.c_double()
        nbytes = ctypes.c_double()
        check(lib.nnc_hip_profile_entry(i, name, 128, ctypes.byref(launches), ctypes.byref(ms)),
              "nnc_hip_profile_entry")
        check(lib.nnc_hip_profile_work(i, ctypes.byref(flops), ctypes.byref(nbytes)), "nnc_hip_profile_work")
        out.append({"name": name.value.decode(), "launches": launches.value, "ms": ms.value,
                    "flops": flops.value, "bytes": nbytes.value})
    return out
