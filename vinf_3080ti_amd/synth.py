"""Seeded synthetic GGUF weights for tests and benchmarks.

Two generators:
  synthetic_rows   the reference tests' recipe (test_phase30_cuda_qmatvec.py:45-57): random bytes per block,
                   every fp16 scale field overwritten by uniform(0.001, 0.05).
  baseline_rows    the benchmark recipe: random bytes (uniform codes, grid indices, sign bits and 6-bit/8-bit
                   sub-block scales over all encodings) with every fp16 scale field set to fp16(|N(0, 1e-3)|).
Both return a numpy uint8 array of rows*row_bytes bytes. `torch_baseline_rows` builds the same
distribution directly in device memory for the large benchmark shapes.
"""
from __future__ import annotations

import numpy as np

from .gguf_types import F16_FIELDS, GGUFTensorType, traits


def _blocks(tensor_type: int, rows: int, cols: int, rng: np.random.Generator) -> np.ndarray:
    bs, ts = traits(tensor_type)
    nblk = rows * cols // bs
    return rng.integers(0, 256, size=(nblk, ts), dtype=np.uint8)


def _set_f16(blocks: np.ndarray, tensor_type: int, values: np.ndarray) -> None:
    for k, off in enumerate(F16_FIELDS[GGUFTensorType(tensor_type)]):
        blocks[:, off : off + 2] = values[:, k].astype("<f2").view(np.uint8).reshape(-1, 2)


def synthetic_rows(tensor_type: int, rows: int, cols: int, seed: int | np.random.Generator = 0) -> np.ndarray:
    rng = seed if isinstance(seed, np.random.Generator) else np.random.default_rng(seed)
    t = GGUFTensorType(tensor_type)
    if t is GGUFTensorType.F32:
        return rng.uniform(-1, 1, rows * cols).astype("<f4").view(np.uint8)
    if t is GGUFTensorType.F16:
        return rng.uniform(-1, 1, rows * cols).astype("<f2").view(np.uint8)
    blocks = _blocks(t, rows, cols, rng)
    n = len(F16_FIELDS[t])
    _set_f16(blocks, t, rng.uniform(0.001, 0.05, size=(blocks.shape[0], n)))
    return blocks.reshape(-1)


def baseline_rows(tensor_type: int, rows: int, cols: int, seed: int | np.random.Generator = 20261201) -> np.ndarray:
    rng = seed if isinstance(seed, np.random.Generator) else np.random.default_rng(seed)
    t = GGUFTensorType(tensor_type)
    if t is GGUFTensorType.F32:
        return rng.standard_normal(rows * cols).astype("<f4").view(np.uint8)
    if t is GGUFTensorType.F16:
        return rng.standard_normal(rows * cols).astype("<f2").view(np.uint8)
    blocks = _blocks(t, rows, cols, rng)
    n = len(F16_FIELDS[t])
    _set_f16(blocks, t, np.abs(rng.normal(0.0, 1e-3, size=(blocks.shape[0], n))))
    return blocks.reshape(-1)


def torch_baseline_rows(tensor_type: int, rows: int, cols: int, seed: int, device, pad: int = 256):
    """baseline_rows' distribution generated on `device` (torch uint8, nbytes + pad, pad bytes zero)."""
    import torch

    t = GGUFTensorType(tensor_type)
    if t in (GGUFTensorType.F32, GGUFTensorType.F16):
        raise ValueError("torch_baseline_rows generates quantized types only")
    bs, ts = traits(t)
    nblk = rows * cols // bs
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    buf = torch.zeros(nblk * ts + pad, dtype=torch.uint8, device=device)
    body = buf[: nblk * ts]
    body.copy_(torch.randint(0, 256, (nblk * ts,), dtype=torch.uint8, device=device, generator=gen))
    if t in F16_FIELDS:
        blocks = body.view(nblk, ts)
        for off in F16_FIELDS[t]:
            d = torch.randn(nblk, device=device, generator=gen).mul_(1e-3).abs_().to(torch.float16)
            blocks[:, off : off + 2] = d.view(torch.uint8).view(nblk, 2)
    return buf
