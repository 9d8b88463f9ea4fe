"""The prefill contraction's work plan (G16Plan in vq_gemm16_impl.h), checked on the host for 1568 shapes x CU
counts x modes: walking every workgroup's ranges as the kernels do, each unit is covered exactly once and wg_of
names its owner; a part of a tile is only ever written for tiles the reduction visits (>= t0), at slot k <
maxseg, in slot order; and the workspace layout holds every slot. No GPU: hipcc compiles the check as host code."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_g16_plan_covers_every_unit_once(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    exe = tmp_path / "g16_plan_check"
    src = ROOT / "tests" / "g16_plan_check.hip"
    inc = ROOT / "vinf_3080ti_amd" / "csrc"
    build = subprocess.run([hipcc, "-O1", "-std=c++20", f"-I{inc}", "-I" + str(ROOT / "include"), str(src), "-o",
                            str(exe)], capture_output=True, text=True, timeout=300)
    assert build.returncode == 0, build.stdout + build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout
    assert "bad 0" in run.stdout and "hybrid 0" not in run.stdout, run.stdout
