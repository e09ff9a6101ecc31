"""Python side of libnnc_costmodel.so, the cost-model runtime.

The library implements the nnc_* ABI like libnnc_hip.so but prices each
call on an analytic MI355X timeline instead of computing it (the
counterpart of the reference's runtime/x86/costmodel.c, selected there with
NNC_RUNTIME_IMPL=costmodel, codegen/x86_emitters/build_files.py:50-81).
`estimate(prog)` runs a compiled program's call sequence through it and
returns the simulated step time and the per-kernel table, so a compiler
pass can compare alternatives without a GPU.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from pathlib import Path

from . import abi

LIB = Path(__file__).resolve().parent / "lib" / "libnnc_costmodel.so"
_lib = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and bind libnnc_costmodel.so. Its per-call trace is off
    (NNC_COSTMODEL_QUIET) unless the caller set that variable."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB
    if not p.exists():
        raise FileNotFoundError(f"{p} is not built (python -c 'import __graft_entry__ as g; g.build()')")
    os.environ.setdefault("NNC_COSTMODEL_QUIET", "1")
    lib = ctypes.CDLL(str(p))
    abi.bind(lib)
    lib.nnc_costmodel_reset.argtypes, lib.nnc_costmodel_reset.restype = [], None
    lib.nnc_costmodel_elapsed_us.argtypes, lib.nnc_costmodel_elapsed_us.restype = [], ctypes.c_double
    lib.nnc_costmodel_kernel_count.argtypes, lib.nnc_costmodel_kernel_count.restype = [], ctypes.c_int
    lib.nnc_costmodel_kernel.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int64),
                                         ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                         ctypes.POINTER(ctypes.c_double)]
    lib.nnc_costmodel_kernel.restype = ctypes.c_int
    for name in ("nnc_hip_stream_fork", "nnc_hip_stream_join"):
        getattr(lib, name).argtypes, getattr(lib, name).restype = [], ctypes.c_int
    lib.nnc_hip_stream_select.argtypes, lib.nnc_hip_stream_select.restype = [ctypes.c_int], ctypes.c_int
    lib.nnc_hip_transfer.argtypes = [abi.TP, abi.TP]
    _lib = lib
    return lib


@dataclass
class KernelCost:
    name: str
    launches: int
    us: float
    flops: float
    bytes: float


@dataclass
class Estimate:
    step_us: float
    kernels: list[KernelCost]

    def by_name(self) -> dict[str, KernelCost]:
        return {k.name: k for k in self.kernels}


def table(lib: ctypes.CDLL | None = None) -> list[KernelCost]:
    lib = lib or load()
    out = []
    name = ctypes.create_string_buffer(128)
    n, us, fl, by = ctypes.c_int64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    for i in range(lib.nnc_costmodel_kernel_count()):
        lib.nnc_costmodel_kernel(i, name, 128, ctypes.byref(n), ctypes.byref(us), ctypes.byref(fl), ctypes.byref(by))
        out.append(KernelCost(name.value.decode(), n.value, us.value, fl.value, by.value))
    return out


def estimate(prog, lib: ctypes.CDLL | None = None) -> Estimate:
    """One nnc_run() of `prog` (a compiler Program) on the model: simulated
    step time in microseconds and the per-kernel table."""
    from .compiler import Executor
    lib = lib or load()
    ex = Executor(prog, device=False, lib=lib)
    lib.nnc_costmodel_reset()
    ex.run()
    est = Estimate(lib.nnc_costmodel_elapsed_us(), table(lib))
    ex.close()
    return est
