"""Name-keyed device runtime of the quantized-matvec path (drop-in for vinf's CUDA runtime on this path).

`Runtime` mirrors the method surface of the reference's `_cuda_qwen_runtime.Runtime` that the qwen35
forward pass uses around its matvecs (/root/reference/engine/csrc/megakernel/qwen_runtime.cu:2602-2677):
upload/free/has/tensor_info/device_bytes/mem_info, alloc/zero/write/read/copy/buffer_ptr/buffer_elem,
qmv/matvec, argmax/argmax_rows, set_gemm_min_rows, synchronize. `HipWeightRuntime` mirrors the Python
wrapper `CudaWeightRuntime` (src/vinf/cuda/qwen_runtime.py:47-116), so
`QwenGpuExecutor(..., runtime=HipWeightRuntime())` reaches these kernels for every qmv.

Device memory is held in torch tensors (plumbing only); every computation is a call into libvq_hip.so
on torch's current HIP stream. Errors follow the reference: KeyError for unknown names, ValueError for
bad shapes/sizes/types, TypeError for an fp16 buffer where fp32 is needed, RuntimeError("<ctx> failed:
<device error>") for device errors.
"""
from __future__ import annotations

import contextlib
import ctypes
import math
from dataclasses import dataclass
from typing import Sequence

import numpy as np
import torch

from . import _lib
from .gguf_types import HIP_MATVEC_TYPES, GGUFTensorType, traits

MAX_TOKENS = 8  # tokens per matvec launch (kMaxTokens, qwen_runtime.cu:572)
MAX_ARGMAX_ROWS = 256  # kMaxArgmaxRows (qwen_runtime.cu:573)
_PAD = 256  # every weight allocation carries >= 16 readable bytes past its end (qwen_runtime.cu:1366-1367)


@dataclass
class _Tensor:
    data: torch.Tensor  # uint8, nbytes + padding
    type: int
    rows: int
    cols: int
    row_bytes: int
    nbytes: int
    home: str = "own"  # where the bytes live: "own" allocation, "arena", or "group:<id>"
    streamed: bool = False  # uploaded with resident=False (served from HBM all the same)


@dataclass
class _Region:
    """A device allocation that resident uploads are carved from (the weight arena, or one weight group)."""

    data: torch.Tensor  # uint8
    used: int = 0
    names: list[str] | None = None

    def carve(self, padded: int) -> torch.Tensor | None:
        if self.used + padded > self.data.numel():
            return None
        view = self.data[self.used : self.used + padded]
        self.used += padded
        return view


# Granule that weight-group sizes are rounded to (the reference rounds to its VMM granularity).
WEIGHT_GRANULE = 2 << 20


@dataclass
class _Buffer:
    data: torch.Tensor  # float32 or float16
    elem: int


def _check_upload_args(name: str, nbytes_given: int, type_id: int, cols: int, rows: int) -> tuple[int, int]:
    """Validation of Runtime_upload (qwen_runtime.cu:1338-1357). Returns (row_bytes, nbytes)."""
    try:
        bs, ts = traits(type_id)
    except ValueError:
        raise ValueError(f"unsupported GGUF tensor type id {type_id} for HIP matvec") from None
    if cols <= 0 or rows <= 0 or cols % bs != 0:
        raise ValueError(f"{name}: cols={cols} must be a positive multiple of the block size")
    row_bytes = cols // bs * ts
    nbytes = row_bytes * rows
    if nbytes_given != nbytes:
        raise ValueError(f"{name}: got {nbytes_given} bytes, expected {nbytes}")
    return row_bytes, nbytes


def _check_qmv_args(name: str, cols: int, ntok: int) -> None:
    """Validation of Runtime_qmv (qwen_runtime.cu:1865-1868)."""
    if ntok < 1:
        raise ValueError("ntok must be positive")
    if cols % 32 != 0:
        raise ValueError(f"{name}: matvec cols must be a multiple of 32")


class Runtime:
    """Persistent device store of raw GGUF tensors and fp32 buffers, keyed by name."""

    def __init__(self, iq3s_grid: bytes | None = None, device: int | None = None) -> None:
        if not torch.cuda.is_available():
            raise RuntimeError("Runtime needs a ROCm GPU: torch.cuda.is_available() is False")
        self._lib = _lib.load()
        self.device = torch.device("cuda", torch.cuda.current_device() if device is None else device)
        with torch.cuda.device(self.device):
            _lib.check(self._lib.vq_init(), "vq_init")
            if iq3s_grid is not None:
                grid = bytes(iq3s_grid)
                if len(grid) != 512 * 4:
                    raise ValueError("iq3s_grid must be 2048 bytes (512 entries x 4 values)")
                _lib.check(self._lib.vq_set_iq3s_grid(grid), "vq_set_iq3s_grid")
        self.tensors: dict[str, _Tensor] = {}
        self.buffers: dict[str, _Buffer] = {}
        self._argmax_out = torch.empty(MAX_ARGMAX_ROWS, dtype=torch.int32, device=self.device)
        self._ws = torch.empty(0, dtype=torch.uint8, device=self.device)
        self.gemm_min_rows = 0
        self.batch_invariant = False
        self.gemm_f16_activations = False
        self._paging: tuple[torch.Tensor, int, int, int] | None = None
        self._segments: list[tuple[int, int, int, int]] = []
        # Resident-weight memory: an optional arena and the executor's per-layer weight groups. Nothing streams
        # over PCIe here, so the stream order only records which uploads were requested as streamed.
        self._arena: _Region | None = None
        self._weight_space: int | None = None
        self._groups: list[_Region] = []
        self._stream_order: list[str] = []

    # ---- helpers ----------------------------------------------------------------------------------
    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _workspace(self, nbytes: int) -> torch.Tensor:
        """Device scratch for packed activations / argmax keys, grown on demand and reused (stream-ordered)."""
        if self._ws.numel() < nbytes:
            self._ws = torch.empty(max(nbytes, 2 * self._ws.numel()), dtype=torch.uint8, device=self.device)
        return self._ws

    def _logits_scratch(self, n: int) -> torch.Tensor:
        """fp32 logits of the batch-invariant argmax when the caller keeps none: grown on demand and reused
        (separate from the workspace, which the matvec itself may use)."""
        buf = getattr(self, "_logits", None)
        if buf is None or buf.numel() < n:
            buf = self._logits = torch.empty(n, dtype=torch.float32, device=self.device)
        return buf

    def _tensor(self, name: str) -> _Tensor:
        t = self.tensors.get(name)
        if t is None:
            raise KeyError(f"weight tensor {name} is not loaded")
        return t

    def _any_buffer(self, name: str) -> _Buffer:
        b = self.buffers.get(name)
        if b is None:
            raise KeyError(f"device buffer {name} is not allocated")
        return b

    def _f32_buffer(self, name: str, min_n: int) -> torch.Tensor:
        """find_buffer (qwen_runtime.cu:1206-1223)."""
        b = self._any_buffer(name)
        if b.elem != 4:
            raise TypeError(f"device buffer {name} is fp16 (KV cache), not fp32")
        if b.data.numel() < min_n:
            raise ValueError(f"device buffer {name} has {b.data.numel()} floats, need {min_n}")
        return b.data

    # ---- weights ----------------------------------------------------------------------------------
    def upload(self, name: str, data, type_id: int, cols: int, rows: int, resident: bool = True, group: int = -1) -> None:
        """Copy raw GGUF blocks to the device (Runtime_upload, qwen_runtime.cu:1338-1409).

        Every tensor is resident in HBM: `resident=False` (pinned-host streaming on the 12 GB card) is recorded
        (set_stream_order accepts such names) but the bytes go to HBM all the same. group >= 0 places the tensor
        in that weight group's allocation, else the arena (set_arena) while it has room, else its own allocation.
        """
        if group >= 0 and group >= len(self._groups):
            raise ValueError(f"unknown weight group {group}")
        # The views are released on every exit: a caller's mapping (upload_gguf_tensor) can then be closed
        # even when this raises.
        with memoryview(data) as src, src.cast("B") as view:
            row_bytes, nbytes = _check_upload_args(name, view.nbytes, int(type_id), int(cols), int(rows))
            host = torch.frombuffer(bytearray(view), dtype=torch.uint8)
        padded = (nbytes + 16 + _PAD - 1) // _PAD * _PAD
        dev, home = None, "own"
        if group >= 0:
            dev, home = self._groups[group].carve(padded), f"group:{group}"
            if dev is None:
                raise ValueError(f"weight group {group} has no room for {name}")
            self._groups[group].names.append(name)
        elif self._arena is not None:
            dev = self._arena.carve(padded)
            home = "arena" if dev is not None else "own"
        if dev is None:
            dev = torch.empty(padded, dtype=torch.uint8, device=self.device)
        self.tensors.pop(name, None)
        dev[nbytes:].zero_()
        dev[:nbytes].copy_(host)
        self.tensors[name] = _Tensor(dev, int(type_id), int(rows), int(cols), row_bytes, nbytes, home,
                                     streamed=not resident)

    def upload_device(self, name: str, data: torch.Tensor, type_id: int, cols: int, rows: int) -> None:
        """Register device-resident raw blocks (uint8 tensor of >= nbytes + 16 bytes) without a host copy."""
        if data.device != self.device or data.dtype != torch.uint8 or not data.is_contiguous():
            raise ValueError(f"{name}: expected a contiguous uint8 tensor on {self.device}")
        try:
            bs, ts = traits(type_id)
        except ValueError:
            raise ValueError(f"unsupported GGUF tensor type id {type_id} for HIP matvec") from None
        if cols <= 0 or rows <= 0 or cols % bs != 0:
            raise ValueError(f"{name}: cols={cols} must be a positive multiple of the block size")
        row_bytes = cols // bs * ts
        nbytes = row_bytes * rows
        if data.numel() < nbytes + 16:
            raise ValueError(f"{name}: device tensor needs {nbytes + 16} bytes (16 bytes of tail padding)")
        if data.data_ptr() % 16:
            raise ValueError(f"{name}: device tensor must be 16-byte aligned")
        self.tensors[name] = _Tensor(data, int(type_id), int(rows), int(cols), row_bytes, nbytes)

    def free(self, name: str) -> None:
        if name not in self.tensors:
            raise KeyError(name)
        del self.tensors[name]

    def has(self, name: str) -> bool:
        return name in self.tensors

    def device_bytes(self) -> int:
        return sum(t.nbytes for t in self.tensors.values())

    # ---- resident-weight memory (the executor's load path) -----------------------------------------------
    # The reference plans weights for a 12 GB card: an arena for resident tensors, VMM weight groups that can be
    # demoted to pinned host memory, a ring that streams the rest over PCIe (qwen_runtime.cu:1436-1810). On one
    # MI355X (288 GB) the whole model stays in HBM, so these calls keep their meaning for resident weights and
    # report zero for everything that would stream.
    def set_arena(self, nbytes: int) -> None:
        """One allocation that later resident uploads are carved from, 256-byte aligned (qwen_runtime.cu:1486-1500).
        RuntimeError while a tensor lives in the current arena; 0 drops it."""
        busy = next((n for n, t in self.tensors.items() if t.home == "arena"), None)
        if busy is not None:
            raise RuntimeError(f"arena is in use by {busy}")
        self._arena = None
        if nbytes > 0:
            self._arena = _Region(torch.empty(int(nbytes), dtype=torch.uint8, device=self.device))

    def vmm_granularity(self) -> int:
        return WEIGHT_GRANULE

    def set_weight_space(self, nbytes: int) -> None:
        """Capacity of the weight groups added next (qwen_runtime.cu:1713-1726)."""
        if self._groups:
            raise RuntimeError("weight space in use")
        self._weight_space = int(nbytes)

    def add_weight_group(self, nbytes: int) -> int:
        """A device allocation of nbytes rounded up to the granule, for one layer's tensors; returns its id
        (qwen_runtime.cu:1728-1744)."""
        if self._weight_space is None:
            raise RuntimeError("set_weight_space first")
        size = -(-int(nbytes) // WEIGHT_GRANULE) * WEIGHT_GRANULE
        if sum(g.data.numel() for g in self._groups) + size > self._weight_space:
            raise ValueError("weight space exhausted")
        self._groups.append(_Region(torch.empty(size, dtype=torch.uint8, device=self.device), names=[]))
        return len(self._groups) - 1

    def weight_groups(self) -> list[tuple[int, bool, list[str]]]:
        """[(bytes, mapped, tensor names)] per group (qwen_runtime.cu:1794-1811); every group stays mapped."""
        return [(g.data.numel(), True, list(g.names)) for g in self._groups]

    def _group_id(self, gid: int) -> int:
        if not 0 <= gid < len(self._groups):
            raise ValueError(f"unknown weight group {gid}")
        return gid

    def demote_group(self, gid: int) -> None:
        """Moving a group to pinned host memory (qwen_runtime.cu:1746-1770) is PCIe streaming, which this
        runtime does not do: every weight stays in HBM. Raises RuntimeError for a known group."""
        self._group_id(gid)
        raise RuntimeError("demote_group: weights stay resident in HBM (no host streaming on this runtime)")

    def promote_group(self, gid: int) -> bool:
        """Groups are never demoted, so each one is already resident (qwen_runtime.cu:1772-1792)."""
        self._group_id(gid)
        return True

    def set_stream_order(self, names, slots: int) -> None:
        """Order of the streamed tensors (qwen_runtime.cu:1523-1593). Each name must be a tensor uploaded with
        resident=False (ValueError otherwise, or when it repeats); those are in HBM here, so no ring is built."""
        if isinstance(names, (str, bytes)) or not hasattr(names, "__iter__"):
            raise TypeError("names must be a sequence of str")
        order: list[str] = []
        for n in names:
            if not isinstance(n, str):
                raise TypeError("names must be a sequence of str")
            t = self.tensors.get(n)
            if t is None or not t.streamed:
                raise ValueError(f"{n} is not a loaded streamed tensor")
            if n in order:
                raise ValueError(f"{n} appears twice in the stream order")
            order.append(n)
        self._stream_order = order

    def reserve_ring(self, slot_bytes: int, slots: int) -> None:
        """Ring slots for streamed weights (qwen_runtime.cu:1595-1614): none are needed, nothing streams."""
        if slot_bytes < 0 or slots < 0:
            raise ValueError("reserve_ring sizes must be >= 0")

    def vram_bytes(self) -> int:
        """Device memory this runtime holds: arena, weight groups, tensors in their own allocations, buffers and
        the matvec workspace (qwen_runtime.cu:1436-1446)."""
        total = sum(g.data.numel() for g in self._groups)
        total += self._arena.data.numel() if self._arena is not None else 0
        total += sum(t.data.numel() for t in self.tensors.values() if t.home == "own")
        return total + self.buffer_bytes() + self._ws.numel()

    def buffer_bytes(self) -> int:
        return sum(b.data.numel() * b.elem for b in self.buffers.values())

    def staging_bytes(self) -> int:
        return 0  # no staging buffers or ring slots

    def pinned_bytes(self) -> int:
        return 0  # no tensor lives in host memory

    def streamed_bytes(self) -> int:
        return 0  # nothing crosses PCIe on the matvec path

    def map_range(self, name: str, offset: int, n: int) -> bool:
        """Buffers are backed in full when allocated (alloc's virtual flag reserves nothing lazily), so every
        in-bounds range is mapped (qwen_runtime.cu:1671-1680)."""
        self._range_check(name, offset, n, "map_range")
        return True

    def unmap_range(self, name: str, offset: int, n: int) -> None:
        self._range_check(name, offset, n, "unmap_range")

    def map_cost(self, name: str, offset: int, n: int) -> int:
        self._any_buffer(name)
        return 0

    def _range_check(self, name: str, offset: int, n: int, what: str) -> None:
        b = self._any_buffer(name)
        if offset < 0 or n < 0 or offset + n > b.data.numel():
            raise ValueError(f"{what} out of bounds")

    def tensor_info(self, name: str) -> tuple[int, int, int, int, int, int, bool]:
        """(device_address, gguf_type, rows, cols, row_bytes, nbytes, resident) (qwen_runtime.cu:1460-1473)."""
        t = self._tensor(name)
        return (t.data.data_ptr(), t.type, t.rows, t.cols, t.row_bytes, t.nbytes, True)

    def mem_info(self) -> tuple[int, int]:
        return torch.cuda.mem_get_info(self.device)

    # ---- buffers ----------------------------------------------------------------------------------
    def alloc(self, name: str, n: int, elem: int = 4, virtual: bool = False) -> None:
        """Zeroed device buffer of n elements (Runtime_alloc, qwen_runtime.cu:1616-1650)."""
        if n <= 0:
            raise ValueError(f"buffer {name} size must be positive")
        if elem not in (4, 2):
            raise ValueError("element size must be 4 (fp32) or 2 (fp16)")
        dtype = torch.float32 if elem == 4 else torch.float16
        self.buffers[name] = _Buffer(torch.zeros(int(n), dtype=dtype, device=self.device), elem)

    def zero(self, name: str) -> None:
        buf = self._any_buffer(name)
        _lib.check(self._lib.vq_zero(buf.data.data_ptr(), buf.data.numel() * buf.elem, self._stream()), "zero")

    def write(self, name: str, data, offset: int = 0) -> None:
        b = self._any_buffer(name)
        view = memoryview(data).cast("B")
        if offset < 0 or view.nbytes % b.elem or offset + view.nbytes // b.elem > b.data.numel():
            raise ValueError(f"write to {name}: bad offset/size for {b.elem}-byte elements")
        host = torch.frombuffer(bytearray(view), dtype=b.data.dtype)
        b.data[offset : offset + host.numel()].copy_(host)

    def read(self, name: str, n: int = -1, offset: int = 0) -> bytes:
        b = self._any_buffer(name)
        avail = b.data.numel()
        if offset < 0 or offset > avail:
            raise ValueError("bad read offset")
        count = avail - offset if n < 0 else n
        if offset + count > avail:
            raise ValueError(f"read of {count} elements exceeds buffer {name}")
        return b.data[offset : offset + count].cpu().numpy().tobytes()

    def buffer_ptr(self, name: str) -> tuple[int, int]:
        b = self._f32_buffer(name, 0)
        return (b.data_ptr(), b.numel())

    def buffer_elem(self, name: str) -> int:
        return self._any_buffer(name).elem

    def buffer_tensor(self, name: str) -> torch.Tensor:
        """The torch tensor behind a buffer (for zero-copy interop)."""
        return self._any_buffer(name).data

    # ---- the hot path -------------------------------------------------------------------------------
    def qmv(self, weight: str, x: str, y: str, ntok: int = 1) -> None:
        """y[t] = W x[t] for t < ntok, asynchronous on the current stream (Runtime_qmv, qwen_runtime.cu:1860-1912)."""
        if ntok < 1:
            raise ValueError("ntok must be positive")
        t = self._tensor(weight)
        _check_qmv_args(weight, t.cols, ntok)
        xb = self._f32_buffer(x, t.cols * ntok)
        yb = self._f32_buffer(y, t.rows * ntok)
        self._qmv_ptrs(t, xb.data_ptr(), yb.data_ptr(), ntok)

    def _qmv_ptrs(self, t: _Tensor, x_ptr: int, y_ptr: int, ntok: int) -> None:
        if t.type not in (0, 1) and self.gemm_min_rows > 0 and ntok >= self.gemm_min_rows:
            # Prompt pass: the MFMA contraction (the prefill branch of Runtime_qmv, qwen_runtime.cu:1886-1902):
            # packed activations, then the contraction's own workspace (f16 path of Q2_K-Q6_K, IQ2_XXS/XS/S and
            # IQ3_XXS; 0 bytes otherwise).
            flags = _lib.VQ_GEMM_BATCH_INVARIANT if self.batch_invariant else 0
            ng = self._lib.vq_qgemm_workspace_bytes_ex(t.type, t.rows, t.cols, ntok, flags)
            if self.gemm_f16_activations and ng:
                # The reference's own numerics: fp32 activations rounded to f16 inside the call.
                buf = self._workspace(ng)
                st = self._lib.vq_qgemm_f16x_ws(t.type, t.data.data_ptr(), t.rows, t.cols, x_ptr, ntok, y_ptr,
                                                buf.data_ptr(), ng, flags, self._stream())
                _lib.check(st, "qgemm launch")
                return
            nx = (self._lib.vq_xpack_bytes(t.cols, ntok) + 255) // 256 * 256
            buf = self._workspace(nx + ng)
            xp = buf.data_ptr()
            _lib.check(self._lib.vq_pack_x(x_ptr, ntok, t.cols, xp, self._stream()), "pack_x")
            st = self._lib.vq_qgemm_ws_ex(t.type, t.data.data_ptr(), t.rows, t.cols, xp, ntok, y_ptr,
                                          (xp + nx) if ng else None, ng, flags, self._stream())
            _lib.check(st, "qgemm launch")
            return
        if t.type in (0, 1):
            ws = None
            nws = 0
        else:
            nws = self._lib.vq_qmv_workspace_bytes_for(t.type, t.rows, t.cols, ntok)
            ws = self._workspace(nws).data_ptr() if nws else None
        st = self._lib.vq_qmv(t.type, t.data.data_ptr(), t.rows, t.cols, x_ptr, ntok, y_ptr, ws, nws, self._stream())
        _lib.check(st, "qmv launch")

    def qmv_staged(self, weight: str, x: str, y: str, ntok: int = 1, *, x2: str | None = None,
                   norm: str | None = None, eps: float = 1e-6, add: bool = False) -> None:
        """y[t] (+)= W v[t] with the activations staged inside the matvec, as the megakernel's QMV flags do
        (qwen_megakernel.cu:468-551; runtime/instructions.py:179-182): v = silu(x) * x2 when x2 is given, then
        rmsnorm(v) * norm when norm (an F32 tensor or fp32 buffer of cols values) is given; add=True
        accumulates into y. Quantized weights; cols <= 24576 except on the small-batch path (5-16 tokens of
        Q3_K..Q6_K and the IQ types but IQ4_NL, any cols multiple of 256). No counterpart in the per-op runtime,
        whose callers run silu_mul, rmsnorm and add as passes of their own."""
        if ntok < 1:
            raise ValueError("ntok must be positive")
        t = self._tensor(weight)
        if t.type in (0, 1):
            raise ValueError(f"{weight}: qmv_staged needs a quantized weight")
        _check_qmv_args(weight, t.cols, ntok)
        xb = self._f32_buffer(x, t.cols * ntok)
        yb = self._f32_buffer(y, t.rows * ntok)
        flags = _lib.VQ_QMV_ADD if add else 0
        x2p = nwp = None
        if x2 is not None:
            flags |= _lib.VQ_QMV_SILU_MUL
            x2p = self._f32_buffer(x2, t.cols * ntok).data_ptr()
        if norm is not None:
            flags |= _lib.VQ_QMV_NORM
            if norm in self.tensors:
                nt = self._tensor(norm)
                if nt.type != 0 or nt.rows * nt.cols != t.cols:
                    raise ValueError(f"{norm}: norm weights must be an F32 tensor of {t.cols} values")
                nwp = nt.data.data_ptr()
            else:
                nwp = self._f32_buffer(norm, t.cols).data_ptr()
        # 5-16 tokens of the f16 small-batch types stage inside that kernel (vq_qmv_staged_ws, with the RMS
        # prepass and partial sums in the runtime's workspace); other calls stream (vq_qmv_staged).
        nws = self._lib.vq_qmv_staged_workspace_bytes(t.type, t.rows, t.cols, ntok)
        ws = self._workspace(nws) if nws else None
        st = self._lib.vq_qmv_staged_ws(t.type, t.data.data_ptr(), t.rows, t.cols, xb.data_ptr(), x2p, nwp,
                                        float(eps), flags, ntok, yb.data_ptr(), ws.data_ptr() if ws is not None else None,
                                        nws, self._stream())
        _lib.check(st, "qmv_staged launch")

    # ---- ops around the matvec (the reference runtime's elementwise / norm ops) ------------------------------
    def _f32_weight(self, name: str, n: int) -> torch.Tensor:
        """find_f32_weight: an uploaded F32 tensor of n values."""
        t = self._tensor(name)
        if t.type != 0 or t.rows * t.cols != n:
            raise ValueError(f"{name}: expected an F32 tensor of {n} values")
        return t.data

    def rmsnorm(self, x: str, w: str, y: str, n: int, eps: float = 1e-6, groups: int = 1) -> None:
        """y[g] = x[g] * rsqrt(mean(x[g]^2) + eps) * w for each of `groups` rows of n (Runtime_rmsnorm,
        qwen_runtime.cu:36-44,1914-1925); w an F32 tensor; y may be x."""
        if n < 1 or groups < 1:
            raise ValueError("n and groups must be positive")
        xb, yb = self._f32_buffer(x, n * groups), self._f32_buffer(y, n * groups)
        wt = self._f32_weight(w, n)
        _lib.check(self._lib.vq_rmsnorm(xb.data_ptr(), wt.data_ptr(), None, yb.data_ptr(), n, groups, float(eps),
                                        self._stream()), "rmsnorm")

    def gated_rmsnorm(self, x: str, w: str, z: str, y: str, n: int, eps: float, groups: int) -> None:
        """y = rmsnorm(x) * w * silu(z) per group of n (Runtime_gated_rmsnorm, qwen_runtime.cu:46-52,1927-1939)."""
        if n < 1 or groups < 1:
            raise ValueError("n and groups must be positive")
        xb, zb = self._f32_buffer(x, n * groups), self._f32_buffer(z, n * groups)
        yb = self._f32_buffer(y, n * groups)
        wt = self._f32_weight(w, n)
        _lib.check(self._lib.vq_rmsnorm(xb.data_ptr(), wt.data_ptr(), zb.data_ptr(), yb.data_ptr(), n, groups,
                                        float(eps), self._stream()), "gated_rmsnorm")

    def _binary(self, op: int, a: str, b: str, out: str, n: int) -> None:
        """binary_op (qwen_runtime.cu:1941-1954)."""
        if n < 0:
            raise ValueError("n must be non-negative")
        ab, bb, ob = self._f32_buffer(a, n), self._f32_buffer(b, n), self._f32_buffer(out, n)
        _lib.check(self._lib.vq_binary(op, ab.data_ptr(), bb.data_ptr(), ob.data_ptr(), n, self._stream()),
                   "elementwise")

    def add(self, a: str, b: str, out: str, n: int) -> None:
        self._binary(0, a, b, out, n)

    def silu_mul(self, gate: str, up: str, out: str, n: int) -> None:
        self._binary(1, gate, up, out, n)

    def sigmoid_mul(self, x: str, gate: str, out: str, n: int) -> None:
        self._binary(2, x, gate, out, n)

    def split_gated_q(self, raw: str, q: str, gate: str, heads: int, hd: int) -> None:
        """Per head, raw [query(hd), gate(hd)] -> q, gate (Runtime_split_gated_q, qwen_runtime.cu:70-76)."""
        if heads < 1 or hd < 1:
            raise ValueError("heads and hd must be positive")
        n = heads * hd
        rb, qb, gb = self._f32_buffer(raw, 2 * n), self._f32_buffer(q, n), self._f32_buffer(gate, n)
        _lib.check(self._lib.vq_split_gated_q(rb.data_ptr(), qb.data_ptr(), gb.data_ptr(), heads, hd, self._stream()),
                   "split_gated_q")

    def rope(self, x: str, heads: int, hd: int, rot: int, pos: int, base: float = 10000.0, ntok: int = 1) -> None:
        """NeoX partial RoPE in place over the first rot dims of each head, token t at position pos + t
        (Runtime_rope, qwen_runtime.cu:81-92)."""
        if rot <= 0 or rot % 2 != 0 or rot > hd:
            raise ValueError(f"invalid rotary dim {rot}")
        if ntok < 1:
            raise ValueError("ntok must be positive")
        if heads < 1 or pos < 0:
            raise ValueError("heads must be positive and pos non-negative")
        xb = self._f32_buffer(x, heads * hd * ntok)
        _lib.check(self._lib.vq_rope(xb.data_ptr(), ntok, heads, hd, rot, pos, float(base), self._stream()), "rope")

    def kv_append(self, k: str, v: str, kc: str, vc: str, kv_heads: int, max_seq: int, hd: int, pos: int,
                  ntok: int = 1) -> None:
        """k, v [ntok][kv_heads][hd] into the caches [kv_heads][max_seq][hd] at positions pos .. pos + ntok - 1
        (Runtime_kv_append, qwen_runtime.cu:115-128); fp16 caches are written rounded to nearest."""
        if ntok < 1 or pos < 0 or pos + ntok > max_seq:
            raise ValueError(f"positions [{pos}, {pos + ntok}) outside KV cache of {max_seq}")
        n, cache = kv_heads * hd * ntok, kv_heads * hd * max_seq
        kb, vb = self._f32_buffer(k, n), self._f32_buffer(v, n)
        kcb, vcb = self._any_buffer(kc), self._any_buffer(vc)
        for name, b in ((kc, kcb), (vc, vcb)):
            if b.data.numel() < cache:
                raise ValueError(f"device buffer {name} has {b.data.numel()} values, need {cache}")
        if kcb.elem != vcb.elem:
            raise TypeError("K and V caches differ in precision")
        _lib.check(self._lib.vq_kv_append(kb.data_ptr(), vb.data_ptr(), kcb.data.data_ptr(), vcb.data.data_ptr(),
                                          kcb.elem, ntok, kv_heads, max_seq, hd, pos, self._stream()), "kv_append")

    def attention(self, q: str, kc: str, vc: str, out: str, heads: int, kv_heads: int, hd: int, max_seq: int,
                  seq_len: int, ntok: int = 1, bidirectional: int = 0, window: int = 0) -> None:
        """GQA attention of ntok query tokens over contiguous KV caches (Runtime_attention, qwen_runtime.cu:
        128-162); token t sees seq_len + t positions (causal) or seq_len + ntok - 1 (bidirectional), the last
        `window` of them when window > 0."""
        if kv_heads <= 0 or heads % kv_heads != 0:
            raise ValueError("heads must be divisible by kv_heads")
        if ntok < 1 or seq_len <= 0 or seq_len + ntok - 1 > max_seq:
            raise ValueError(f"invalid seq_len {seq_len} for {ntok} tokens")
        n, cache = heads * hd * ntok, kv_heads * hd * max_seq
        qb = self._f32_buffer(q, n)
        kcb, vcb = self._any_buffer(kc), self._any_buffer(vc)
        for name, b in ((kc, kcb), (vc, vcb)):
            if b.data.numel() < cache:
                raise ValueError(f"device buffer {name} has {b.data.numel()} values, need {cache}")
        ob = self._f32_buffer(out, n)
        if kcb.elem != vcb.elem:
            raise TypeError("K and V caches differ in precision")
        if self._tiled_attention(ntok):
            _lib.check(self._lib.vq_attention_tiled(qb.data_ptr(), kcb.data.data_ptr(), vcb.data.data_ptr(),
                                                    ob.data_ptr(), kcb.elem, heads, kv_heads, hd, max_seq, seq_len, ntok,
                                                    int(bidirectional), int(window), self._stream()), "attention")
            return
        nws = self._lib.vq_attention_workspace_bytes(heads, kv_heads, hd, seq_len, ntok, int(window))
        ws = self._workspace(nws).data_ptr() if nws else None
        _lib.check(self._lib.vq_attention_ws(qb.data_ptr(), kcb.data.data_ptr(), vcb.data.data_ptr(), ob.data_ptr(),
                                             kcb.elem, heads, kv_heads, hd, max_seq, seq_len, ntok, int(bidirectional),
                                             int(window), ws, nws, self._stream()), "attention")

    def conv_update(self, x: str, state: str, w: str, out: str, channels: int, K: int, ntok: int = 1,
                    snap: str | None = None, write_state: int = 1) -> None:
        """Causal depthwise conv + SiLU stepping through ntok tokens, state [channels][K] updated in place unless
        write_state is 0 (a verification pass), w an F32 tensor [channels][K] (Runtime_conv_update,
        qwen_runtime.cu:397-426,2078-2100)."""
        if ntok < 1:
            raise ValueError("ntok must be positive")
        xb = self._f32_buffer(x, channels * ntok)
        sb = self._f32_buffer(state, channels * K)
        ob = self._f32_buffer(out, channels * ntok)
        wt = self._f32_weight(w, channels * K)
        snp = self._f32_buffer(snap, channels * K * (ntok - 1)).data_ptr() if snap is not None else None
        if K > _lib.VQ_CONV_MAX_K:
            raise ValueError(f"conv kernel size {K} > {_lib.VQ_CONV_MAX_K}")
        _lib.check(self._lib.vq_conv_update(xb.data_ptr(), sb.data_ptr(), wt.data_ptr(), ob.data_ptr(), channels, K,
                                            ntok, snp, int(bool(write_state)), self._stream()), "conv_update")

    def gated_delta(self, conv: str, b: str, a: str, ssm_a: str, dt: str, state: str, out: str, key_heads: int,
                    value_heads: int, kd: int, vd: int, eps: float, head_order: int, ntok: int = 1,
                    snap: str | None = None, write_state: int = 1) -> None:
        """Gated delta rule stepping through ntok tokens, fp32 state [vh][kd][vd] in place (unless write_state
        is 0); ssm_a and dt are F32 tensors of value_heads values (Runtime_gated_delta, qwen_runtime.cu:433-567,
        2139-2165)."""
        if key_heads <= 0 or value_heads % key_heads != 0:
            raise ValueError("value heads must be a multiple of key heads")
        if ntok < 1:
            raise ValueError("ntok must be positive")
        conv_dim = 2 * key_heads * kd + value_heads * vd
        state_n = value_heads * kd * vd
        cb = self._f32_buffer(conv, conv_dim * ntok)
        bb, ab = self._f32_buffer(b, value_heads * ntok), self._f32_buffer(a, value_heads * ntok)
        sb, ob = self._f32_buffer(state, state_n), self._f32_buffer(out, value_heads * vd * ntok)
        sa, dtt = self._f32_weight(ssm_a, value_heads), self._f32_weight(dt, value_heads)
        snp = self._f32_buffer(snap, state_n * (ntok - 1)).data_ptr() if snap is not None else None
        _lib.check(self._lib.vq_gated_delta(cb.data_ptr(), bb.data_ptr(), ab.data_ptr(), sa.data_ptr(), dtt.data_ptr(),
                                            sb.data_ptr(), 4, ob.data_ptr(), key_heads, value_heads, kd, vd, float(eps),
                                            int(head_order), ntok, snp, int(bool(write_state)), self._stream()),
                   "gated_delta")

    def concat_rows(self, dst: str, a: str, b: str, rows: int, width: int) -> None:
        """dst[r] = [a[r] | b[r]] for rows of width floats (Runtime_concat_rows, qwen_runtime.cu:2567-2587)."""
        if rows < 0 or width < 0:
            raise ValueError("rows and width must be non-negative")
        n = rows * width
        ab, bb, db = self._f32_buffer(a, n), self._f32_buffer(b, n), self._f32_buffer(dst, 2 * n)
        _lib.check(self._lib.vq_concat_rows(db.data_ptr(), ab.data_ptr(), bb.data_ptr(), rows, width, self._stream()),
                   "concat_rows")

    def zero_range(self, name: str, offset: int, n: int) -> None:
        """Clear n elements of a buffer from offset (Runtime_zero_range, qwen_runtime.cu:2589-2600)."""
        buf = self._any_buffer(name)
        if offset < 0 or n < 0 or offset + n > buf.data.numel():
            raise ValueError("zero_range out of bounds")
        _lib.check(self._lib.vq_zero(buf.data.data_ptr() + offset * buf.elem, n * buf.elem, self._stream()),
                   "zero_range")

    # ---- multi-sequence passes (paged KV caches, per-slot recurrent state) --------------------------------------
    def set_paging(self, page_table: str, page_size: int, pages_per_seq: int, max_slots: int) -> None:
        """KV caches of the *_seg ops are page pools [page][kv_head][page_size][hd]; the buffer page_table holds
        int32 page ids [max_slots][pages_per_seq] (Runtime_set_paging, qwen_runtime.cu:2333-2350)."""
        if page_size < 1 or pages_per_seq < 1 or max_slots < 1:
            raise ValueError("invalid paging shape")
        pt = self._f32_buffer(page_table, pages_per_seq * max_slots)
        self._paging = (pt, int(page_size), int(pages_per_seq), int(max_slots))

    def set_segments(self, segments) -> int:
        """Row layout of the next *_seg ops: [(slot, pos0, rows[, row0]), ...], rows of a segment being
        consecutive positions of one sequence slot, stacked in order unless row0 places them. Returns the row
        after the last segment (Runtime_set_segments, qwen_runtime.cu:2352-2385)."""
        if self._paging is None:
            raise RuntimeError("set_paging first")
        _, page, pps, slots = self._paging
        table: list[tuple[int, int, int, int]] = []
        row0 = 0
        for seg in segments:
            if not 3 <= len(seg) <= 4:
                raise TypeError("a segment is (slot, pos0, rows[, row0])")
            slot, pos0, rows = (int(v) for v in seg[:3])
            if len(seg) == 4 and int(seg[3]) >= 0:
                row0 = int(seg[3])
            if slot < 0 or slot >= slots or pos0 < 0 or rows < 1 or pos0 + rows > page * pps:
                raise ValueError(f"segment ({slot}, {pos0}, {rows}) outside the paged context")
            table.append((slot, pos0, rows, row0))
            row0 += rows
        if not table:
            raise ValueError("no segments")
        self._segments = table
        return row0

    def _seg_ready(self) -> list[tuple[int, int, int, int]]:
        if not self._segments or self._paging is None:
            raise RuntimeError("set_paging and set_segments must be called before *_seg ops")
        return self._segments

    def _seg_rows(self) -> int:
        return max(r0 + n for _, _, n, r0 in self._seg_ready())

    def _seg_chunks(self):
        """The segment table as int32 arrays of at most VQ_MAX_SEGMENTS segments (one launch each)."""
        segs = self._seg_ready()
        for i in range(0, len(segs), _lib.VQ_MAX_SEGMENTS):
            part = segs[i:i + _lib.VQ_MAX_SEGMENTS]
            yield (ctypes.c_int32 * (4 * len(part)))(*[v for sg in part for v in sg]), len(part)

    def _kv_pair(self, kc: str, vc: str, min_n: int) -> tuple[_Buffer, _Buffer]:
        """find_kv_buffer for a K/V cache pair of one precision (qwen_runtime.cu:1226-1248)."""
        kcb, vcb = self._any_buffer(kc), self._any_buffer(vc)
        for name, buf in ((kc, kcb), (vc, vcb)):
            if buf.data.numel() < min_n:
                raise ValueError(f"device buffer {name} has {buf.data.numel()} values, need {min_n}")
        if kcb.elem != vcb.elem:
            raise TypeError("K and V caches differ in precision")
        return kcb, vcb

    def rope_seg(self, x: str, heads: int, hd: int, rot: int, base: float) -> None:
        """NeoX RoPE with each segment's positions (Runtime_rope_seg, qwen_runtime.cu:2400-2417)."""
        self._seg_ready()
        if rot <= 0 or rot % 2 != 0 or rot > hd:
            raise ValueError(f"invalid rotary dim {rot}")
        xb = self._f32_buffer(x, heads * hd * self._seg_rows())
        for arr, n in self._seg_chunks():
            _lib.check(self._lib.vq_rope_seg(xb.data_ptr(), arr, n, heads, hd, rot, float(base), self._stream()),
                       "rope_seg")

    def kv_append_seg(self, k: str, v: str, kc: str, vc: str, kv_heads: int, hd: int) -> None:
        """Append each segment's K/V rows to its sequence's pages (Runtime_kv_append_seg, qwen_runtime.cu:
        2419-2447)."""
        self._seg_ready()
        rowsz = kv_heads * hd
        kb, vb = self._f32_buffer(k, rowsz * self._seg_rows()), self._f32_buffer(v, rowsz * self._seg_rows())
        kcb, vcb = self._kv_pair(kc, vc, rowsz)
        pt, page, pps, _ = self._paging
        for arr, n in self._seg_chunks():
            _lib.check(self._lib.vq_kv_append_seg(kb.data_ptr(), vb.data_ptr(), kcb.data.data_ptr(), vcb.data.data_ptr(),
                                                  kcb.elem, arr, n, kv_heads, hd, pt.data_ptr(), page, pps,
                                                  self._stream()), "kv_append_seg")

    def attention_seg(self, q: str, kc: str, vc: str, out: str, heads: int, kv_heads: int, hd: int) -> None:
        """Causal attention of each segment over its own pages (Runtime_attention_seg, qwen_runtime.cu:
        2449-2478)."""
        self._seg_ready()
        if kv_heads <= 0 or heads % kv_heads != 0:
            raise ValueError("heads must be divisible by kv_heads")
        rowsz = heads * hd
        qb = self._f32_buffer(q, rowsz * self._seg_rows())
        kcb, vcb = self._kv_pair(kc, vc, 1)
        ob = self._f32_buffer(out, rowsz * self._seg_rows())
        pt, page, pps, _ = self._paging
        tiled = self._tiled_attention(max(r for _, _, r, _ in self._segments))
        for arr, n in self._seg_chunks():
            if tiled:  # prompt rows in the pass, or batch-invariant mode
                _lib.check(self._lib.vq_attention_seg_tiled(qb.data_ptr(), kcb.data.data_ptr(), vcb.data.data_ptr(),
                                                            ob.data_ptr(), kcb.elem, arr, n, heads, kv_heads, hd,
                                                            pt.data_ptr(), page, pps, self._stream()), "attention_seg")
                continue
            nws = self._lib.vq_attention_seg_workspace_bytes(arr, n, heads, kv_heads, hd)
            ws = self._workspace(nws).data_ptr() if nws else None
            _lib.check(self._lib.vq_attention_seg_ws(qb.data_ptr(), kcb.data.data_ptr(), vcb.data.data_ptr(),
                                                     ob.data_ptr(), kcb.elem, arr, n, heads, kv_heads, hd,
                                                     pt.data_ptr(), page, pps, ws, nws, self._stream()),
                       "attention_seg")

    def conv_update_seg(self, x: str, state: str, w: str, out: str, channels: int, K: int, snap: str | None = None,
                        write_state: int = 1) -> None:
        """Per-segment causal conv over the slot's state [slots][channels][K]; snapshots need a single segment
        (Runtime_conv_update_seg, qwen_runtime.cu:2480-2511)."""
        segs = self._seg_ready()
        if K > _lib.VQ_CONV_MAX_K:
            raise ValueError(f"conv kernel size {K} > {_lib.VQ_CONV_MAX_K}")
        ntok, stride = self._seg_rows(), channels * K
        xb = self._f32_buffer(x, channels * ntok)
        sb = self._f32_buffer(state, stride * self._paging[3])
        ob = self._f32_buffer(out, channels * ntok)
        wt = self._f32_weight(w, stride)
        snp = None
        if snap is not None:
            if len(segs) != 1:
                raise ValueError("snapshots need a single-segment pass")
            snp = self._f32_buffer(snap, stride * (ntok - 1)).data_ptr()
        for arr, n in self._seg_chunks():
            _lib.check(self._lib.vq_conv_update_seg(xb.data_ptr(), sb.data_ptr(), wt.data_ptr(), ob.data_ptr(), channels,
                                                    K, arr, n, snp, int(bool(write_state)), self._stream()),
                       "conv_update_seg")

    def gated_delta_seg(self, conv: str, b: str, a: str, ssm_a: str, dt: str, state: str, out: str, key_heads: int,
                        value_heads: int, kd: int, vd: int, eps: float, head_order: int, snap: str | None = None,
                        write_state: int = 1) -> None:
        """Per-segment gated delta rule over the slot's state [slots][vh][kd][vd], fp32 or fp16 (fp16: no
        snapshots) (Runtime_gated_delta_seg, qwen_runtime.cu:2513-2565)."""
        segs = self._seg_ready()
        if key_heads <= 0 or value_heads % key_heads != 0:
            raise ValueError("value heads must be a multiple of key heads")
        ntok = self._seg_rows()
        conv_dim = 2 * key_heads * kd + value_heads * vd
        state_n = value_heads * kd * vd
        cb = self._f32_buffer(conv, conv_dim * ntok)
        bb, ab = self._f32_buffer(b, value_heads * ntok), self._f32_buffer(a, value_heads * ntok)
        sbuf = self._any_buffer(state)
        if sbuf.data.numel() < state_n * self._paging[3]:
            raise ValueError(f"device buffer {state} has {sbuf.data.numel()} values, need {state_n * self._paging[3]}")
        ob = self._f32_buffer(out, value_heads * vd * ntok)
        sa, dtt = self._f32_weight(ssm_a, value_heads), self._f32_weight(dt, value_heads)
        snp = None
        if snap is not None:
            if sbuf.elem == 2:
                raise ValueError("fp16 SSM state does not support snapshots")
            if len(segs) != 1:
                raise ValueError("snapshots need a single-segment pass")
            snp = self._f32_buffer(snap, state_n * (ntok - 1)).data_ptr()
        for arr, n in self._seg_chunks():
            _lib.check(self._lib.vq_gated_delta_seg(cb.data_ptr(), bb.data_ptr(), ab.data_ptr(), sa.data_ptr(),
                                                    dtt.data_ptr(), sbuf.data.data_ptr(), sbuf.elem, ob.data_ptr(),
                                                    key_heads, value_heads, kd, vd, float(eps), int(head_order), arr, n,
                                                    snp, int(bool(write_state)), self._stream()), "gated_delta_seg")

    def copy(self, dst: str, dst_off: int, src: str, src_off: int, n: int) -> None:
        """dst[dst_off:+n] = src[src_off:+n] in elements, buffers of one precision (Runtime_copy,
        qwen_runtime.cu:2200-2218); asynchronous on the current stream."""
        if dst_off < 0 or src_off < 0 or n < 0:
            raise ValueError("offsets and count must be non-negative")
        db, sb = self._any_buffer(dst), self._any_buffer(src)
        if db.elem != sb.elem:
            raise TypeError("copy between buffers of different precision")
        if dst_off + n > db.data.numel() or src_off + n > sb.data.numel():
            raise ValueError(f"copy out of bounds ({dst} <- {src})")
        if n:
            db.data[dst_off:dst_off + n].copy_(sb.data[src_off:src_off + n], non_blocking=True)

    def qmv_group(self, weights: Sequence[str], x: str, ys: Sequence[str], ntok: int = 1) -> None:
        """ys[k][t] = W_k x[t] for up to 4 quantized weights of one width that read the same input, in one
        launch (a layer's gate/up or q/k/v; one quantized type, or one type plus Q8_0 small tensors). Same
        results as one qmv per weight; no counterpart in the reference's per-op runtime, whose callers issue
        one qmv each (qwen_gpu.py:865-867)."""
        if not 1 <= len(weights) <= 4 or len(weights) != len(ys):
            raise ValueError("qmv_group takes 1 to 4 weights and as many outputs")
        if ntok < 1:
            raise ValueError("ntok must be positive")
        ts = [self._tensor(w) for w in weights]
        t0 = ts[0]
        if any(t.cols != t0.cols or t.type in (0, 1) for t in ts):
            raise ValueError("qmv_group weights must be quantized and share cols")
        _check_qmv_args(weights[0], t0.cols, ntok)
        if self.gemm_min_rows > 0 and ntok >= self.gemm_min_rows:  # prompt (or batch-invariant) passes: as qmv
            for w, y in zip(weights, ys):
                self.qmv(w, x, y, ntok)
            return
        xb = self._f32_buffer(x, t0.cols * ntok)
        yb = [self._f32_buffer(y, t.rows * ntok) for y, t in zip(ys, ts)]
        n = len(ts)
        wa = (ctypes.c_void_p * n)(*[t.data.data_ptr() for t in ts])
        ra = (ctypes.c_int * n)(*[t.rows for t in ts])
        ya = (ctypes.c_void_p * n)(*[b.data_ptr() for b in yb])
        if any(t.type != t0.type for t in ts):
            # Mixed types (Q5_K projections with Q8_0 small tensors, or Q5_K with Q6_K): one launch.
            ta = (ctypes.c_int * n)(*[t.type for t in ts])
            st = self._lib.vq_qmv_group_mixed_f32(n, ta, wa, ra, ya, t0.cols, xb.data_ptr(), ntok, self._stream())
        else:
            # One type: the streaming group launch, or for small batches the MFMA paths qmv would take (5-16
            # tokens of Q3_K..Q6_K as one launch over all the matrices).
            nws = self._lib.vq_qmv_group_workspace_bytes(t0.type, n, ra, t0.cols, ntok)
            ws = self._workspace(nws).data_ptr() if nws else None
            st = self._lib.vq_qmv_group_ws(t0.type, n, wa, ra, ya, t0.cols, xb.data_ptr(), ntok, ws, nws,
                                           self._stream())
        _lib.check(st, "qmv_group launch")

    def lmhead_argmax(self, weight: str, x: str, ntok: int = 1, logits: str | None = None) -> list[int]:
        """argmax_r (W x[t])[r] for t < ntok, fused with the matvec (ties -> lowest row, NaN never wins);
        the logits are written to `logits` only if given. Equals qmv + argmax_rows (qwen_runtime.cu:1860-1912,
        2181-2197) without re-reading the logits, like the megakernel's fused argmax
        (qwen_megakernel.cu:552-606,800-829)."""
        if not 1 <= ntok <= MAX_ARGMAX_ROWS:
            raise ValueError(f"ntok must be in [1, {MAX_ARGMAX_ROWS}]")
        t = self._tensor(weight)
        if t.type in (0, 1):
            raise ValueError(f"{weight}: lmhead_argmax needs a quantized weight")
        _check_qmv_args(weight, t.cols, ntok)
        xb = self._f32_buffer(x, t.cols * ntok)
        if self.batch_invariant:  # the matvec on the invariant path, then the row argmax
            yt = (self._f32_buffer(logits, t.rows * ntok) if logits is not None
                  else self._logits_scratch(t.rows * ntok))
            self._qmv_ptrs(t, xb.data_ptr(), yt.data_ptr(), ntok)
            _lib.check(self._lib.vq_argmax_rows(yt.data_ptr(), t.rows, ntok, self._argmax_out.data_ptr(),
                                                self._stream()), "argmax_rows")
            return [int(v) for v in self._argmax_out[:ntok].tolist()]
        lp = self._f32_buffer(logits, t.rows * ntok).data_ptr() if logits is not None else None
        nws = self._lib.vq_lmhead_argmax_workspace_bytes(t.type, t.rows, t.cols, ntok)
        ws = self._workspace(nws)
        st = self._lib.vq_lmhead_argmax(t.type, t.data.data_ptr(), t.rows, t.cols, xb.data_ptr(), ntok,
                                        self._argmax_out.data_ptr(), lp, ws.data_ptr(), nws, self._stream())
        _lib.check(st, "lmhead_argmax")
        return [int(v) for v in self._argmax_out[:ntok].tolist()]

    def qmv_tensor(self, weight: str, x: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
        """Tensor form: x [ntok, cols] fp32 on the device -> y [ntok, rows] fp32."""
        t = self._tensor(weight)
        if x.dim() == 1:
            x = x.unsqueeze(0)
        ntok = x.shape[0]
        _check_qmv_args(weight, t.cols, ntok)
        if x.shape[1] != t.cols or x.dtype != torch.float32 or x.device != self.device:
            raise ValueError(f"{weight}: x must be float32 [ntok, {t.cols}] on {self.device}")
        x = x.contiguous()
        if x.data_ptr() % 16:  # the kernels read activations with 16-byte loads
            x = x.clone()
        if y is None:
            y = torch.empty(ntok, t.rows, dtype=torch.float32, device=self.device)
        self._qmv_ptrs(t, x.data_ptr(), y.data_ptr(), ntok)
        return y

    def matvec(self, name: str, x: bytes) -> bytes:
        """Synchronous debug matvec: fp32 bytes in, fp32 bytes out (Runtime_matvec, qwen_runtime.cu:2280-2315)."""
        t = self.tensors.get(name)
        if t is None:
            raise KeyError(f"{name} is not resident on the GPU")
        view = memoryview(x).cast("B")
        if view.nbytes != t.cols * 4:
            raise ValueError(f"{name}: x has {view.nbytes} bytes, expected {t.cols} float32")
        xd = torch.frombuffer(bytearray(view), dtype=torch.float32).to(self.device)
        y = self.qmv_tensor(name, xd)
        torch.cuda.synchronize(self.device)
        return y.cpu().numpy().tobytes()

    def argmax(self, name: str, n: int) -> int:
        """Index of the largest of the first n floats; ties -> lowest index (Runtime_argmax, :2167-2179)."""
        xb = self._f32_buffer(name, n)
        _lib.check(self._lib.vq_argmax_rows(xb.data_ptr(), n, 1, self._argmax_out.data_ptr(), self._stream()), "argmax")
        return int(self._argmax_out[0].item())

    def argmax_rows(self, name: str, n: int, ntok: int) -> list[int]:
        """Row-wise argmax of ntok rows of n floats (Runtime_argmax_rows, :2181-2197)."""
        if ntok < 1 or ntok > MAX_ARGMAX_ROWS:
            raise ValueError(f"ntok must be in [1, {MAX_ARGMAX_ROWS}]")
        xb = self._f32_buffer(name, n * ntok)
        _lib.check(self._lib.vq_argmax_rows(xb.data_ptr(), n, ntok, self._argmax_out.data_ptr(), self._stream()),
                   "argmax_rows")
        return [int(v) for v in self._argmax_out[:ntok].tolist()]

    def set_gemm_min_rows(self, n: int) -> None:
        """qmv calls with ntok >= n take the MFMA prefill contraction (0 = never) (qwen_runtime.cu:2324-2330)."""
        if n < 0:
            raise ValueError("gemm_min_rows must be >= 0")
        self.gemm_min_rows = int(n)

    def set_batch_invariant(self, on: bool = True) -> None:
        """Every pass on the kernels whose per-row results do not depend on the other rows of the pass: qmv through
        the prompt contraction with a K split fixed by the matrix (gemm_min_rows = 1), attention through the tiled
        kernel. The reference's --batch-invariant mode (qwen_cli.py:47-49; it sets gemm_min_rows to 1 for every
        pass, qwen_gpu.py:738-744): slower for a lone request, and a request's outputs never depend on what runs
        beside it. Off restores gemm_min_rows = 0."""
        self.batch_invariant = bool(on)
        self.gemm_min_rows = 1 if on else 0

    def set_gemm_f16_activations(self, on: bool = True) -> None:
        """Prompt-pass contractions (ntok >= gemm_min_rows) on the f16 path's types with the activations rounded to
        f16, one MFMA per product: the reference's tensor-core numerics (f32_to_f16_rows_kernel + vinf_qgemm_kernel,
        qwen_runtime.cu:657-739), ~1.3-1.45x faster at 512 tokens. Off (the default): activations as the CPU path's
        int8 codes in two f16 halves, matching the CPU path to rel-L2 1e-5. Other types take the int8 contraction
        either way. No counterpart call in the reference, whose GPU prompt pass always rounds to f16."""
        self.gemm_f16_activations = bool(on)

    def _tiled_attention(self, rows: int) -> bool:
        return self.batch_invariant or (self.gemm_min_rows > 0 and rows >= self.gemm_min_rows)

    def synchronize(self) -> None:
        torch.cuda.synchronize(self.device)


def iq3s_grid_bytes() -> bytes:
    """The 2048-byte IQ3_S codebook the reference passes to Runtime() (cuda/qwen_runtime.py:41-44)."""
    from .tables import table

    return table("iq3s_grid")


class HipWeightRuntime:
    """Drop-in for CudaWeightRuntime (src/vinf/cuda/qwen_runtime.py:47-116): the executor's `runtime=` object.

    It owns a `Runtime` built with the IQ3_S codebook and adds the host-list conveniences the executor uses
    (float lists in and out, GGUF uploads); every other attribute is the `Runtime` method of the same name.
    """

    def __init__(self, device: int | None = None) -> None:
        self._rt = Runtime(iq3s_grid_bytes(), device)

    def upload_gguf_tensor(self, gguf, name: str, *, device_name: str | None = None, resident: bool = True,
                           group: int = -1) -> int:
        """Upload one tensor's raw blocks from the file mapping (cuda/qwen_runtime.py:68-86) and return its
        byte size. The innermost GGUF dimension is the row length; the outer ones multiply into the row count.
        A type without a HIP matvec raises UnsupportedModelError before anything is mapped."""
        from .gguf import UnsupportedModelError

        info = gguf.tensors[name]
        kind = info.tensor_type
        if int(kind) not in HIP_MATVEC_TYPES:
            raise UnsupportedModelError(f"{name}: no HIP matvec for {kind.name}")
        row_len, *outer = info.dimensions
        with contextlib.ExitStack() as cleanup:
            handle, mapping, view = gguf.mmap_tensor(name)
            # Unwound last-in first-out: the view is released before its mapping and file are closed.
            cleanup.callback(handle.close)
            cleanup.callback(mapping.close)
            cleanup.callback(view.release)
            self._rt.upload(device_name or name, view, int(kind), row_len, math.prod(outer), resident, group)
        return info.nbytes

    def upload_raw(self, name: str, data, tensor_type: GGUFTensorType, cols: int, rows: int, *,
                   resident: bool = True) -> None:
        if int(tensor_type) not in HIP_MATVEC_TYPES:
            raise ValueError(f"{name}: no HIP matvec for type {int(tensor_type)}")
        self._rt.upload(name, data, int(tensor_type), cols, rows, resident)

    def matvec(self, name: str, values: Sequence[float]) -> list[float]:
        """Synchronous W @ values for one host vector, as a list of Python floats."""
        packed = np.ascontiguousarray(values, dtype="<f4").tobytes()
        return np.frombuffer(self._rt.matvec(name, packed), dtype="<f4").tolist()

    def read_floats(self, name: str, n: int = -1, offset: int = 0) -> list[float]:
        """A buffer's elements as Python floats; fp16 buffers (KV caches) are widened exactly."""
        width = "<f2" if self._rt.buffer_elem(name) == 2 else "<f4"
        return np.frombuffer(self._rt.read(name, n, offset), dtype=width).tolist()

    def write_floats(self, name: str, values, offset: int = 0) -> None:
        self._rt.write(name, np.ascontiguousarray(values, dtype="<f4").tobytes(), offset)

    def __getattr__(self, name: str):
        return getattr(self._rt, name)
