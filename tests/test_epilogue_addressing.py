"""Addressing of C in the short-product GEMM's epilogue (CPU only, no GPU call).

gemm_ws_k stores four consecutive columns per thread and adds beta * C,
where C is a bias row (C[j]) or a full matrix (C[i*N + j]). Written per
element through a helper that branches on the C mode, hipcc 7.2 compiled
elements 1..3 of the bias case with the matrix row's base (C + i*N), which
reads past the end of a bias of N floats: a GPU memory fault on a 512-row
product. The kernel now picks the C row once; this checks, in the gfx950
code of the built library, that the four C loads of every gemm_ws_k
instantiation are addressed from one base register pair.
"""

from __future__ import annotations

import re
import shutil

import pytest

from test_finish_order import ROCM_BIN, _library_kernels

C_LOAD = re.compile(r"^\s*global_load_dword\s+v\d+,\s*(v\[\d+:\d+\]),\s*off\b")
ADDR = re.compile(r"^\s*v_lshl_add_u64\s+(v\[\d+:\d+\]),\s*(v\[\d+:\d+\]),\s*2,\s*(v\[\d+:\d+\]|s\[\d+:\d+\])")


def c_load_bases(lines: list[str]) -> list[str]:
    """For each C load (global_load_dword, in layout order), the base pair
    of the v_lshl_add_u64 that last wrote its address before it."""
    bases = []
    for i, line in enumerate(lines):
        m = C_LOAD.match(line)
        if not m:
            continue
        base = None
        for prev in reversed(lines[:i]):
            a = ADDR.match(prev)
            if a and a.group(1) == m.group(1):
                base = a.group(3)
                break
        bases.append(base)
    return bases


def check_one_base(lines: list[str]) -> None:
    bases = c_load_bases(lines)
    assert len(bases) == 4, f"{len(bases)} C loads, expected 4"
    assert None not in bases and len(set(bases)) == 1, f"C loads from different bases: {bases}"


def test_check_rejects_per_element_bases():
    """The miscompiled form: element 0 from C's own base, elements 1..3
    from registers that another path set to the matrix row's base."""
    good = []
    for e in range(4):
        good += [f"v_lshl_add_u64 v[10:11], v[6:7], 2, v[8:9]",
                 f"global_load_dword v3, v[10:11], off offset:{4 * e}"]
    check_one_base(good)
    bad = list(good)
    bad[4] = "v_lshl_add_u64 v[10:11], v[6:7], 2, v[2:3]"
    with pytest.raises(AssertionError):
        check_one_base(bad)
    with pytest.raises(AssertionError):
        check_one_base(good[:6])


@pytest.mark.skipif(not (ROCM_BIN / "llvm-objdump").exists() or not shutil.which("objcopy"),
                    reason="ROCm llvm-objdump or objcopy not installed")
def test_gemm_ws_c_loads_share_one_base(tmp_path, pkg):
    from nnc_py_amd import runtime
    if not runtime.LIB_PATH.exists():
        pytest.fail("libnnc_hip.so is not built: run __graft_entry__.build()")
    kernels = {k: v for k, v in _library_kernels(runtime.LIB_PATH, tmp_path).items()
               if k.startswith("_ZN3nnc9gemm_ws_k")}
    assert len(kernels) == 16, sorted(kernels)  # NS 1..4 x the two operand layouts x2
    for name, lines in kernels.items():
        try:
            check_one_base(lines)
        except AssertionError as e:
            raise AssertionError(f"{name}: {e}") from None
