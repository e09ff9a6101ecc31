"""Host checks of the MFMA engine's stream-K work split (CPU only).

tests/native/streamk_schedule.cpp includes the kernel header and walks the
schedule of every workgroup for a grid of tile / slice / resident-slot
counts, checking that each (tile, K-slice) is computed once, that partial
slots never collide and that the fixup kernel's partial list matches what
the workgroups wrote.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import ROOT

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_streamk_schedule_covers_every_slice_once(tmp_path):
    hipcc = HIPCC
    exe = tmp_path / "streamk_schedule"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17", "-I", str(ROOT / "include"), "-I", str(ROOT / "nnc-py_amd" / "csrc"),
                    str(ROOT / "tests" / "native" / "streamk_schedule.cpp"), "-o", str(exe)],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout + out.stderr
