"""nnc-py_amd: MI355X (gfx950) execution backend for the nnc ONNX->C compiler.

Submodules
  abi       ctypes mirror of the nnc operator ABI (include/nnc_ops.h)
  build     compiles csrc/*.hip into lib/libnnc_hip.so with hipcc (gfx950)
  runtime   loads libnnc_hip.so; device tensors, arena, timing table
  compiler  Compiler(target="mi355x", opt_level=...).compile(...) and the
            host-C code generator whose nnc_run() calls libnnc_hip

The directory name carries a hyphen, so callers import it by path as the
module `nnc_py_amd` (see tests/conftest.py, bench.py, __graft_entry__.py).
"""

__version__ = "0.1.0"
