"""Build the HIP library libvq_hip.so in-tree for gfx950 (hipcc, no JIT cache).

Each translation unit (the C ABI in vq_api.hip and one unit per quantized GGUF type) is compiled to an
object in csrc/_build/ in parallel, then linked into vinf_3080ti_amd/libvq_hip.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = CSRC / "_build"
LIB = PKG / "libvq_hip.so"
INCLUDE = PKG.parent / "include"

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    # Packed fp32 VALU ops stay off: hand-written code and hipcc's own packing both avoid them.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources() -> list[Path]:
    return [CSRC / "vq_api.hip", CSRC / "vq_ops.hip"] + sorted(CSRC.glob("vq_t_*.hip"))


def headers() -> list[Path]:
    return sorted(CSRC.glob("*.h")) + [INCLUDE / "vq.h"]


def hipcc() -> str:
    return str(Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc")


STAMPS_LIB = PKG / "_var" / "libvq_stamps.so"  # timing build (-DVQ_STAMPS): per-workgroup timestamps


def _compile(src: Path, force: bool, build_dir: Path = BUILD, extra: tuple[str, ...] = ()) -> Path:
    obj = build_dir / (src.stem + ".o")
    newest = max(p.stat().st_mtime for p in headers() + [src])
    if force or not obj.exists() or obj.stat().st_mtime < newest:
        tmp = obj.with_suffix(".o.tmp")
        res = subprocess.run([hipcc(), *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(tmp)], stdout=subprocess.PIPE,
                             stderr=subprocess.STDOUT, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}")
        os.replace(tmp, obj)
    return obj


def build(force: bool = True, jobs: int | None = None, verbose: bool = False, stamps: bool = False) -> Path:
    """Compile every translation unit and link LIB. force=False reuses objects newer than their inputs.
    stamps=True builds the timing variant STAMPS_LIB instead (the matvec writes per-workgroup s_memrealtime
    stamps that vq_stamps_read_<type> returns; bench.py --stamps reads them); it never replaces LIB."""
    build_dir = BUILD if not stamps else PKG / "_var" / "obj_stamps"
    lib = LIB if not stamps else STAMPS_LIB
    extra = ("-DVQ_STAMPS",) if stamps else ()
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force, build_dir, extra), srcs))
    if force or not lib.exists() or lib.stat().st_mtime < max(o.stat().st_mtime for o in objs):
        tmp = lib.with_suffix(".so.tmp")
        cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(force="--force" in sys.argv, verbose=True, stamps="--stamps" in sys.argv))
