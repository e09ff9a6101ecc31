"""ctypes mirror of the nnc operator ABI (include/nnc_types.h, include/nnc_ops.h).

The same mirror drives every implementation of the ABI: libnnc_hip.so (device
pointers), and in tests the CPU oracle and the reference runtime (host
pointers). It follows the reference's own ctypes harness
(tests/test_x86_runtime.py:265-272 mirrors the struct the same way).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

DTYPE_FLOAT32 = 0
DTYPE_FLOAT16 = 1
DTYPE_INT32 = 2
DTYPE_INT8 = 3
DTYPE_UINT8 = 4
DTYPE_BOOL = 5
DTYPE_INT64 = 6

# numpy dtype name -> nnc_dtype_t (nnc_types.h)
NUMPY_TO_NNC = {
    "float32": DTYPE_FLOAT32,
    "float16": DTYPE_FLOAT16,
    "int32": DTYPE_INT32,
    "int8": DTYPE_INT8,
    "uint8": DTYPE_UINT8,
    "bool": DTYPE_BOOL,
    "int64": DTYPE_INT64,
}


class Tensor(ctypes.Structure):
    """struct Tensor of nnc_types.h (reference runtime/include/nnc_types.h:27-33)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int),
        ("shape", ctypes.POINTER(ctypes.c_int64)),
        ("ndim", ctypes.c_int),
        ("nbytes", ctypes.c_int64),
    ]


TP = ctypes.POINTER(Tensor)
TPP = ctypes.POINTER(TP)
I64P = ctypes.POINTER(ctypes.c_int64)
I32P = ctypes.POINTER(ctypes.c_int)
F32P = ctypes.POINTER(ctypes.c_float)
c_int = ctypes.c_int
c_float = ctypes.c_float

# Argument lists of every nnc_* entry point (include/nnc_ops.h).
SIGNATURES: dict[str, list] = {
    "nnc_add": [TP, TP, TP],
    "nnc_mul": [TP, TP, TP],
    "nnc_sub": [TP, TP, TP],
    "nnc_div": [TP, TP, TP],
    "nnc_equal": [TP, TP, TP],
    "nnc_and": [TP, TP, TP],
    "nnc_greater": [TP, TP, TP],
    "nnc_or": [TP, TP, TP],
    "nnc_not": [TP, TP],
    "nnc_conv": [TP, TP, TP, TP, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_conv1x1": [TP, TP, TP, TP, c_int, c_int, c_int, c_int],
    "nnc_conv3x3_s1": [TP, TP, TP, TP],
    "nnc_conv7x7_s2": [TP, TP, TP, TP],
    "nnc_conv_relu": [TP, TP, TP, TP, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_conv_relu1x1": [TP, TP, TP, TP, c_int, c_int, c_int, c_int],
    "nnc_conv_relu3x3_s1": [TP, TP, TP, TP],
    "nnc_conv_relu7x7_s2": [TP, TP, TP, TP],
    "nnc_conv_sigmoid": [TP, TP, TP, TP, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_relu": [TP, TP],
    "nnc_sigmoid": [TP, TP],
    "nnc_tanh": [TP, TP],
    "nnc_softmax": [TP, TP, c_int],
    "nnc_clip": [TP, TP, c_float, c_float],
    "nnc_sqrt": [TP, TP],
    "nnc_pow": [TP, TP],
    "nnc_exp": [TP, TP],
    "nnc_log": [TP, TP],
    "nnc_abs": [TP, TP],
    "nnc_neg": [TP, TP],
    "nnc_maxpool2d": [TP, TP, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_avgpool2d": [TP, TP, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_reshape": [TP, TP, I64P, c_int],
    "nnc_flatten": [TP, TP, c_int],
    "nnc_transpose": [TP, TP, I64P, c_int],
    "nnc_squeeze": [TP, TP, c_int],
    "nnc_unsqueeze": [TP, TP, c_int],
    "nnc_tile": [TP, TP, I64P, c_int],
    "nnc_matmul": [TP, TP, TP],
    "nnc_matmul_relu": [TP, TP, TP, TP],
    "nnc_gemm": [TP, TP, TP, TP, c_float, c_float, c_int, c_int],
    "nnc_gemm_nt": [TP, TP, TP, TP, c_float, c_float],
    "nnc_reducemean": [TP, TP, c_int, c_int],
    "nnc_reducesum": [TP, TP, c_int, c_int],
    "nnc_concat": [TPP, TP, c_int, c_int],
    "nnc_batchnorm": [TP, TP, TP, TP, TP, TP, c_float, c_int],
    "nnc_layernorm": [TP, TP, TP, TP, c_int, c_float],
    "nnc_identity": [TP, TP],
    "nnc_split": [TP, TPP, c_int, c_int],
    "nnc_cast": [TP, TP, c_int],
    "nnc_shape": [TP, TP, I64P, c_int],
    "nnc_constantofshape": [TP, c_float, c_int],
    "nnc_expand": [TP, TP, I64P, c_int],
    "nnc_gather": [TP, TP, TP, c_int, c_int],
    "nnc_lstm": [TP, TP, TP, TP, TP, TP, TP, c_int, c_int],
    "nnc_add_relu": [TP, TP, TP],
    "nnc_add_sigmoid": [TP, TP, TP],
}

# The reference runtime defines every name above except this one (the
# reference code generator emits it, no reference runtime defines it).
NOT_IN_REFERENCE = {"nnc_matmul_relu"}

# Fused operators of the mi355x target (include/nnc_hip.h), emitted at O3.
TARGET_SIGNATURES = {
    "nnc_hip_conv_add_relu": [TP, TP, TP, TP, TP, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_hip_conv_packed": [TP, TP, TP, TP, TP, c_int, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_hip_transfer": [TP, TP],
    "nnc_hip_conv_proj": [TP, TP, TP, TP, TP] + [c_int] * 9,
    "nnc_hip_conv_packed_noalloc": [TP, TP, TP, TP, TP, c_int, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_hip_gap_gemm_nt": [TP, TP, TP, TP, c_float, c_float],
    "nnc_hip_conv_maxpool": [TP, TP, TP, TP, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_hip_fused_eltwise": [TPP, c_int, I32P, c_int, F32P, TP],
    "nnc_hip_add_layernorm": [TP, TP, TP, TP, TP, c_int, c_float],
    "nnc_hip_scaled_softmax": [TP, TP, TP, c_int],
    "nnc_hip_attention": [TP, TP, TP, c_int, c_int, c_int, c_int, c_int, c_int, c_int],
    "nnc_hip_transpose_slice": [TP, TP, I64P, c_int, c_int, c_int],
}

# nnc_hip_fused_eltwise's op codes (include/nnc_hip.h NNC_EW_*)
EW_OPS = {"ADD": 0, "SUB": 1, "MUL": 2, "DIV": 3, "ADD_RELU": 4, "ADD_SIGMOID": 5, "RELU": 6, "SIGMOID": 7,
          "TANH": 8, "CLIP": 9}


def bind(lib: ctypes.CDLL, names=None) -> ctypes.CDLL:
    """Attach argtypes/restype for the nnc_* symbols that `lib` exports."""
    table = {**SIGNATURES, **TARGET_SIGNATURES}
    for name in names or table:
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.argtypes = table[name]
        fn.restype = None
    return lib


def make_shape(shape) -> ctypes.Array:
    arr = (ctypes.c_int64 * max(1, len(shape)))()
    for i, s in enumerate(shape):
        arr[i] = int(s)
    return arr


def make_tensor(data_ptr: int, dtype: int, shape, nbytes: int):
    """Return (Tensor, shape_array); keep the array alive as long as the Tensor."""
    sh = make_shape(shape)
    t = Tensor(
        data=ctypes.c_void_p(int(data_ptr)) if data_ptr else None,
        dtype=int(dtype),
        shape=ctypes.cast(sh, I64P),
        ndim=len(shape),
        nbytes=int(nbytes),
    )
    return t, sh


_DECL = re.compile(r"^\s*(?:void|int|void\*|size_t|const char\*)\s*\**\s*(nnc_\w+)\s*\(", re.M)


def declared_symbols(header: Path) -> list[str]:
    """Function names declared in one of include/*.h."""
    text = Path(header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(_DECL.findall(text)))
