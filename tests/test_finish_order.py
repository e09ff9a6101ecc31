"""Instruction order of the in-kernel stream-K finish (CPU only, no GPU call).

A split tile's workgroups store their partials with device-scope (sc1)
buffer stores, wait for them to complete, meet at a barrier and bump the
tile's counter with a relaxed agent-scope atomic; the workgroup that arrives
last waits for the atomic's return, meets its threads at a barrier and reads
the partials back with sc1 loads. That is the AMDGPU memory model's
agent-scope release/acquire without its whole-L2 write-back and invalidate
(nnc-py_amd/csrc/mfma_tile.h states why those are not needed), so the order
of these instructions is what makes the hand-off correct. It is checked in
the gfx950 assembly of

- tests/native/finish_order.hip, a small kernel built on the same helpers,
  compiled here; and
- every kernel of the built libnnc_hip.so that bumps a counter: the gfx950
  code objects are read out of the library's offload bundles and
  disassembled (this library's own code).
"""

from __future__ import annotations

import re
import shutil
import struct
import subprocess
from pathlib import Path

import pytest

from conftest import ROOT

ROCM_BIN = Path("/opt/rocm/llvm/bin")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

PARTIAL_STORE = re.compile(r"^\s*buffer_store_dword(x2|x4)?\s.*\bsc1\b")
PARTIAL_LOAD = re.compile(r"^\s*buffer_load_dword(x2|x4)?\s.*\bsc1\b")
COUNTER_RMW = re.compile(r"^\s*(global|buffer|flat)_atomic_add\w*\s.*\bsc0\b")  # sc0: returns the old value
WAIT_VM0 = re.compile(r"^\s*s_waitcnt\s.*\bvmcnt\(0\)")
BARRIER = re.compile(r"^\s*s_barrier\b")
L2_MAINT = re.compile(r"^\s*buffer_(wbl2|inv)\b")


def check_finish_order(lines: list[str]) -> None:
    """Assert the protocol's order on one kernel's instructions, in the
    order the assembler lays them out. Every hand-off - a counter atomic, or
    the two atomics of finish_arrive_pair between the same two barriers -
    needs its own release and acquire: the device-scope stores before it
    waited for (vmcnt(0)) before a barrier that precedes it, its return
    waited for before the next barrier, and no partial load between it and
    that barrier. A two-level finish chains two hand-offs (a group's sum is
    stored, then handed on)."""
    rmw = [i for i, l in enumerate(lines) if COUNTER_RMW.match(l)]
    assert rmw, "no counter atomic"
    barriers = [i for i, l in enumerate(lines) if BARRIER.match(l)]
    handoffs: list[list[int]] = []
    for i in rmw:
        if handoffs and not any(handoffs[-1][-1] < b < i for b in barriers):
            handoffs[-1].append(i)
        else:
            handoffs.append([i])
    assert all(len(h) <= 2 for h in handoffs), "more than two counter atomics between the same barriers"
    stores = [i for i, l in enumerate(lines) if PARTIAL_STORE.match(l)]
    loads = [i for i, l in enumerate(lines) if PARTIAL_LOAD.match(l)]
    assert loads, "no device-scope partial loads"
    for h in handoffs:
        a, a_last = h[0], h[-1]
        before = [i for i in stores if i < a]
        assert before, "no device-scope partial store before the counter atomic"
        # release: the stores' completion wait, then a barrier, before the atomic
        b1 = max((b for b in barriers if before[-1] < b < a), default=None)
        assert b1 is not None, "no barrier between the partial stores and the counter atomic"
        assert any(WAIT_VM0.match(lines[i]) for i in range(before[-1], b1)), \
            "the partial stores are not waited for (vmcnt(0)) before the barrier"
        # acquire: the atomics have returned before the barrier that releases the readers
        b2 = next((b for b in barriers if b > a_last), None)
        assert b2 is not None, "no barrier after the counter atomic"
        assert any(WAIT_VM0.match(lines[i]) for i in range(a_last, b2)), \
            "the counter atomic's return is not waited for before the barrier"
        # (the window between the two barriers: the code of another path of
        # the kernel may be laid out between a store and this hand-off)
        early = [lines[i].strip() for i in loads if b1 < i < b2]
        assert not early, f"partial loads inside the hand-off: {early[:2]}"
    # the point of the protocol: no whole-L2 write-back or invalidate
    assert not any(L2_MAINT.match(l) for l in lines), "buffer_wbl2 / buffer_inv in the kernel"


def split_kernels(text: str, label: re.Pattern) -> dict[str, list[str]]:
    out: dict[str, list[str]] = {}
    cur = None
    for ln in text.splitlines():
        m = label.match(ln)
        if m:
            cur = m.group(1)
            out[cur] = []
        elif cur is not None:
            out[cur].append(ln)
    return out


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not installed")
def test_finish_protocol_order_in_probe_kernel(tmp_path):
    asm = tmp_path / "finish_order.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "--cuda-device-only", "-S", "-O3", "-std=c++17",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                    "-I", str(ROOT / "include"), "-I", str(ROOT / "nnc-py_amd" / "csrc"),
                    str(ROOT / "tests" / "native" / "finish_order.hip"), "-o", str(asm)],
                   check=True, capture_output=True)
    kernels = split_kernels(asm.read_text(), re.compile(r"^(_Z\w+):"))
    assert len(kernels) == 1
    lines = next(iter(kernels.values()))
    assert sum(1 for l in lines if PARTIAL_STORE.match(l)) == 64
    check_finish_order(lines)


def test_check_rejects_a_missing_wait():
    """check_finish_order fails an order with the stores' completion wait dropped
    or a partial load hoisted above the barrier."""
    good = ["buffer_store_dword v1, v2, s[0:3], 0 offen sc1", "s_waitcnt vmcnt(0)", "s_barrier",
            "global_atomic_add v1, v2, v3, s[4:5] sc0", "s_waitcnt vmcnt(0)", "ds_write_b32 v1, v2",
            "s_waitcnt lgkmcnt(0)", "s_barrier", "buffer_load_dwordx4 v[0:3], v5, s[0:3], 0 offen sc1"]
    check_finish_order(good)
    with pytest.raises(AssertionError):
        check_finish_order(good[:1] + good[2:])  # the stores' wait dropped
    with pytest.raises(AssertionError):
        check_finish_order(good[:4] + good[5:])  # the atomic's wait dropped
    hoisted = good[:4] + [good[8]] + good[4:8]
    with pytest.raises(AssertionError):
        check_finish_order(hoisted)
    with pytest.raises(AssertionError):
        check_finish_order(good[:4] + ["buffer_inv sc1"] + good[4:])
    # two chained hand-offs (a group's sum stored, then handed on): each needs
    # its own release and acquire
    second = ["buffer_store_dwordx4 v[0:3], v5, s[0:3], 0 offen sc1", "s_waitcnt vmcnt(0)", "s_barrier",
              "global_atomic_add v1, v2, v3, s[4:5] sc0", "s_waitcnt vmcnt(0)", "s_barrier",
              "buffer_load_dwordx4 v[0:3], v6, s[0:3], 0 offen sc1"]
    check_finish_order(good + second)
    with pytest.raises(AssertionError):
        check_finish_order(good + second[:1] + second[2:])  # the group sum's store wait dropped
    with pytest.raises(AssertionError):
        check_finish_order(good + second[:4] + second[5:])  # the second atomic's wait dropped
    with pytest.raises(AssertionError):
        check_finish_order(good + second[:4] + [second[6]] + second[4:6])  # a load inside the second hand-off


def _library_kernels(lib: Path, tmp_path: Path) -> dict[str, list[str]]:
    fatbin = tmp_path / "fatbin"
    # input and output named: with the input alone objcopy also rewrites it
    # in place (the library this process may have mapped)
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", str(lib), str(fatbin)], check=True,
                   capture_output=True)
    data = fatbin.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(BUNDLE_MAGIC), data)]
    assert starts, "no offload bundle in .hip_fatbin"
    kernels: dict[str, list[str]] = {}
    for n, s in enumerate(starts):
        # bundle header: magic, entry count, then per entry: offset (from the
        # bundle's start) and size of the code object, triple length, triple
        p = s + len(BUNDLE_MAGIC)
        (count,) = struct.unpack_from("<Q", data, p)
        p += 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", data, p)
            p += 24
            triple = data[p:p + tlen].decode()
            p += tlen
            if triple != TARGET:
                continue
            co = tmp_path / f"co{n}.o"
            co.write_bytes(data[s + off:s + off + size])
            dis = subprocess.run([str(ROCM_BIN / "llvm-objdump"), "-d", "--mcpu=gfx950", str(co)], check=True,
                                 capture_output=True, text=True).stdout
            kernels.update(split_kernels(dis, re.compile(r"^[0-9a-f]+ <(_Z\w+)>:")))
    return kernels


@pytest.mark.skipif(not (ROCM_BIN / "llvm-objdump").exists() or not shutil.which("objcopy"),
                    reason="ROCm llvm-objdump or objcopy not installed")
def test_finish_protocol_order_in_library(tmp_path, pkg):
    from nnc_py_amd import runtime
    if not runtime.LIB_PATH.exists():
        pytest.fail("libnnc_hip.so is not built: run __graft_entry__.build()")
    kernels = _library_kernels(runtime.LIB_PATH, tmp_path)
    finishing = {k: v for k, v in kernels.items() if any(COUNTER_RMW.match(l) for l in v)}
    families = {re.match(r"_ZN3nnc\d+(\w+?_k)", k).group(1) for k in finishing}
    # the GEMM's and the convolution's direct-to-LDS kernels and the short
    # products' kernels finish split tiles in-kernel, the GEMV its K splits,
    # the stem's pool its range boundaries
    assert {"gemm_dma_k", "gemm_ws_k", "gemv_fin_k", "conv_dma_k", "conv_ws_k", "conv_stem_pool_k"} <= families, families
    for name, lines in finishing.items():
        try:
            check_finish_order(lines)
        except AssertionError as e:
            raise AssertionError(f"{name}: {e}") from None
