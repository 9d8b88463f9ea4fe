"""Build the HIP library libvq_hip.so in-tree for gfx950 (hipcc, no JIT cache)."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libvq_hip.so"
SOURCES = [CSRC / "vq_kernels.hip"]
HEADERS = [CSRC / "vq_common.h", CSRC / "vq_decode.h", CSRC / "vq_iq_grids.h", PKG.parent / "include" / "vq.h"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU ops stay off: hand-written code and hipcc's own packing both avoid them.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def build(force: bool = True, verbose: bool = False) -> Path:
    """Compile every source into LIB. force=False skips the compile when LIB is newer than its inputs."""
    if not force and LIB.exists():
        newest = max(p.stat().st_mtime for p in SOURCES + HEADERS)
        if LIB.stat().st_mtime >= newest:
            return LIB
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *map(str, SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
