"""ctypes binding of libvq_hip.so (the C ABI declared in include/vq.h).

Loading fails loudly: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

from .build import LIB

P, I, SZ, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float

# Activation staging flags of vq_qmv_staged (include/vq.h).
VQ_QMV_ADD, VQ_QMV_NORM, VQ_QMV_SILU_MUL = 1, 2, 8

# Sequence ops (include/vq.h).
VQ_MAX_SEGMENTS, VQ_CONV_MAX_K = 64, 8

# name -> (restype, argtypes); every symbol include/vq.h declares.
SIGNATURES: dict[str, tuple[object, list]] = {
    "vq_type_traits": (I, [I, ctypes.POINTER(I), ctypes.POINTER(I)]),
    "vq_row_bytes": (ctypes.c_longlong, [I, I]),
    "vq_status_string": (ctypes.c_char_p, [I]),
    "vq_init": (I, []),
    "vq_set_iq3s_grid": (I, [P]),
    "vq_xpack_bytes": (SZ, [I, I]),
    "vq_qmv_workspace_bytes": (SZ, [I, I]),
    "vq_qmv_workspace_bytes_for": (SZ, [I, I, I, I]),
    "vq_qmv_path": (I, [I, I, I, I, SZ]),
    "vq_qmv_staged": (I, [I, P, I, I, P, P, P, F, I, I, P, P]),
    "vq_qmv_staged_workspace_bytes": (SZ, [I, I, I, I]),
    "vq_qmv_staged_ws": (I, [I, P, I, I, P, P, P, F, I, I, P, P, SZ, P]),
    "vq_rmsnorm": (I, [P, P, P, P, I, I, F, P]),
    "vq_binary": (I, [I, P, P, P, ctypes.c_long, P]),
    "vq_split_gated_q": (I, [P, P, P, I, I, P]),
    "vq_concat_rows": (I, [P, P, P, I, I, P]),
    "vq_zero": (I, [P, SZ, P]),
    "vq_rope": (I, [P, I, I, I, I, I, ctypes.c_double, P]),
    "vq_rope_seg": (I, [P, P, I, I, I, I, ctypes.c_double, P]),
    "vq_kv_append": (I, [P, P, P, P, I, I, I, I, I, I, P]),
    "vq_kv_append_seg": (I, [P, P, P, P, I, P, I, I, I, P, I, I, P]),
    "vq_attention": (I, [P, P, P, P, I, I, I, I, I, I, I, I, I, P]),
    "vq_attention_seg": (I, [P, P, P, P, I, P, I, I, I, I, P, I, I, P]),
    "vq_attention_workspace_bytes": (SZ, [I, I, I, I, I, I]),
    "vq_attention_ws": (I, [P, P, P, P, I, I, I, I, I, I, I, I, I, P, SZ, P]),
    "vq_attention_seg_workspace_bytes": (SZ, [P, I, I, I, I]),
    "vq_attention_seg_ws": (I, [P, P, P, P, I, P, I, I, I, I, P, I, I, P, SZ, P]),
    "vq_attention_tiled": (I, [P, P, P, P, I, I, I, I, I, I, I, I, I, P]),
    "vq_attention_seg_tiled": (I, [P, P, P, P, I, P, I, I, I, I, P, I, I, P]),
    "vq_conv_update": (I, [P, P, P, P, I, I, I, P, I, P]),
    "vq_conv_update_seg": (I, [P, P, P, P, I, I, P, I, P, I, P]),
    "vq_gated_delta": (I, [P, P, P, P, P, P, I, P, I, I, I, I, F, I, I, P, I, P]),
    "vq_gated_delta_seg": (I, [P, P, P, P, P, P, I, P, I, I, I, I, F, I, P, I, P, I, P]),
    "vq_quantize_x": (I, [P, I, I, P, P, P, P]),
    "vq_pack_x": (I, [P, I, I, P, P]),
    "vq_qmv_packed": (I, [I, P, I, I, P, I, P, P]),
    "vq_qmv": (I, [I, P, I, I, P, I, P, P, SZ, P]),
    "vq_qmv_noalloc": (I, [I, P, I, I, P, I, P, P]),
    "vq_int_partials": (I, [I, P, I, I, P, I, P, P]),
    "vq_qmv_group": (I, [I, I, P, P, P, I, P, I, P]),
    "vq_qmv_group_f32": (I, [I, I, P, P, P, I, P, I, P]),
    "vq_qmv_group_workspace_bytes": (SZ, [I, I, P, I, I]),
    "vq_qmv_group_ws": (I, [I, I, P, P, P, I, P, I, P, SZ, P]),
    "vq_qmv_group_mixed_f32": (I, [I, P, P, P, P, I, P, I, P]),
    "vq_qgemm": (I, [I, P, I, I, P, I, P, P]),
    "vq_qgemm_workspace_bytes": (SZ, [I, I, I, I]),
    "vq_qgemm_ws": (I, [I, P, I, I, P, I, P, P, SZ, P]),
    "vq_qgemm_workspace_bytes_ex": (SZ, [I, I, I, I, I]),
    "vq_qgemm_ws_ex": (I, [I, P, I, I, P, I, P, P, SZ, I, P]),
    "vq_qgemm_f16x_ws": (I, [I, P, I, I, P, I, P, P, SZ, I, P]),
    "vq_lmhead_argmax_workspace_bytes": (SZ, [I, I, I, I]),
    "vq_lmhead_argmax": (I, [I, P, I, I, P, I, P, P, P, SZ, P]),
    "vq_dequant_rows": (I, [I, P, I, I, P, P]),
    "vq_argmax_rows": (I, [P, I, I, P, P]),
}

VQ_OK, VQ_ERR_TYPE, VQ_ERR_SHAPE, VQ_ERR_WORKSPACE, VQ_ERR_ARG, VQ_ERR_NOT_INIT, VQ_ERR_TOO_LARGE = 0, -1, -2, -3, -4, -5, -6
VQ_NOALLOC_SCRATCH_BYTES = 32 << 20
VQ_GEMM_BATCH_INVARIANT = 1

_lib: ctypes.CDLL | None = None


class LibraryUnavailableError(RuntimeError):
    """libvq_hip.so is not built or cannot be loaded."""


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load the library (VQ_LIB_PATH overrides the in-tree build, e.g. for tuning variants)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path or os.environ.get("VQ_LIB_PATH") or LIB)
    # torch ships its own HIP runtime; it has to be the process's one before libvq_hip.so resolves its HIP
    # symbols, or the library and torch see two runtimes (vq_init then reports no device).
    import torch  # noqa: F401

    if not p.exists():
        raise LibraryUnavailableError(f"{p} is not built; run `python -m vinf_3080ti_amd.build`")
    try:
        lib = ctypes.CDLL(str(p))
    except OSError as exc:
        raise LibraryUnavailableError(f"cannot load {p}: {exc}") from exc
    variant = path is not None or "VQ_LIB_PATH" in os.environ
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            if variant:  # an older build compared against this one (bench.py --libs): it lacks newer entry points
                continue
            raise
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def status_text(status: int) -> str:
    return load().vq_status_string(status).decode()


def check(status: int, context: str) -> None:
    """Raise the reference's exception types for a non-zero status (qwen_runtime.cu:1100-1103)."""
    if status == VQ_OK:
        return
    if status in (VQ_ERR_TYPE, VQ_ERR_SHAPE, VQ_ERR_ARG):
        raise ValueError(f"{context}: {status_text(status)}")
    raise RuntimeError(f"{context} failed: {status_text(status)}")
