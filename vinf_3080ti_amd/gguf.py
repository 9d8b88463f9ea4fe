"""GGUF container reader: header, metadata, tensor directory and zero-copy views of tensor data.

The layout is the one the reference reads (src/vinf/gguf/parser.py:13-301), GGUF versions 2 and 3, all
little-endian:
- magic b"GGUF", u32 version, u64 tensor count, u64 metadata count;
- metadata entries: string key, u32 value type, value (scalars as their C types, bool as one byte, strings
  as a u64 byte length plus UTF-8 bytes, arrays as a u32 item type, a u64 count and the items);
- tensor entries: string name, u32 dimension count, u64 dimensions (innermost first), u32 tensor type, u64
  offset of the data relative to the data section;
- the data section starts where the header ends, rounded up to `general.alignment` (32 when absent).

Only the header is read (sequentially, through a buffered file); tensor bytes are reached through
`GGUFFile.mmap_tensor`, which maps the file and returns a memoryview of exactly the tensor's blocks, the
zero-copy source `HipWeightRuntime.upload_gguf_tensor` uploads from (cuda/qwen_runtime.py:68-86).
"""
from __future__ import annotations

import math
import mmap
import struct
from dataclasses import dataclass
from enum import IntEnum
from pathlib import Path
from typing import Any, BinaryIO

from .gguf_types import GGUFTensorType

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32


class UnsupportedModelError(ValueError):
    """A file this reader cannot use (the reference's vinf.errors.UnsupportedModelError, errors.py:13)."""


class GGUFValueType(IntEnum):
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


# struct formats of the fixed-size metadata value types
_SCALAR_FMT = {
    GGUFValueType.UINT8: "<B",
    GGUFValueType.INT8: "<b",
    GGUFValueType.UINT16: "<H",
    GGUFValueType.INT16: "<h",
    GGUFValueType.UINT32: "<I",
    GGUFValueType.INT32: "<i",
    GGUFValueType.FLOAT32: "<f",
    GGUFValueType.BOOL: "<?",
    GGUFValueType.UINT64: "<Q",
    GGUFValueType.INT64: "<q",
    GGUFValueType.FLOAT64: "<d",
}

# (block elements, block bytes, quantized) of every tensor type with a known size: the table the reference's
# parser sizes tensors with (parser.py:66-94; its Q8_1 entry is 40 bytes). IQ1_M is a known id without a
# size, as there.
GGUF_TYPE_TRAITS: dict[GGUFTensorType, tuple[int, int, bool]] = {
    GGUFTensorType.F32: (1, 4, False),
    GGUFTensorType.F16: (1, 2, False),
    GGUFTensorType.Q4_0: (32, 18, True),
    GGUFTensorType.Q4_1: (32, 20, True),
    GGUFTensorType.Q5_0: (32, 22, True),
    GGUFTensorType.Q5_1: (32, 24, True),
    GGUFTensorType.Q8_0: (32, 34, True),
    GGUFTensorType.Q8_1: (32, 40, True),
    GGUFTensorType.Q2_K: (256, 84, True),
    GGUFTensorType.Q3_K: (256, 110, True),
    GGUFTensorType.Q4_K: (256, 144, True),
    GGUFTensorType.Q5_K: (256, 176, True),
    GGUFTensorType.Q6_K: (256, 210, True),
    GGUFTensorType.Q8_K: (256, 292, True),
    GGUFTensorType.IQ2_XXS: (256, 66, True),
    GGUFTensorType.IQ2_XS: (256, 74, True),
    GGUFTensorType.IQ3_XXS: (256, 98, True),
    GGUFTensorType.IQ1_S: (256, 50, True),
    GGUFTensorType.IQ4_NL: (32, 18, True),
    GGUFTensorType.IQ3_S: (256, 110, True),
    GGUFTensorType.IQ2_S: (256, 82, True),
    GGUFTensorType.IQ4_XS: (256, 136, True),
    GGUFTensorType.I8: (1, 1, False),
    GGUFTensorType.I16: (1, 2, False),
    GGUFTensorType.I32: (1, 4, False),
    GGUFTensorType.I64: (1, 8, False),
    GGUFTensorType.F64: (1, 8, False),
    GGUFTensorType.BF16: (1, 2, False),
}


@dataclass(frozen=True)
class GGUFMetadataValue:
    type: GGUFValueType
    value: Any


@dataclass(frozen=True)
class GGUFTensorInfo:
    name: str
    dimensions: tuple[int, ...]  # innermost (row length) first
    tensor_type: GGUFTensorType
    relative_offset: int
    absolute_offset: int

    def _trait(self, i: int):
        return GGUF_TYPE_TRAITS[self.tensor_type][i]

    numel = property(lambda self: math.prod(self.dimensions), doc="number of elements")
    block_size = property(lambda self: self._trait(0), doc="elements per block")
    type_size = property(lambda self: self._trait(1), doc="bytes per block")
    is_quantized = property(lambda self: self._trait(2), doc="block-quantized type")

    @property
    def nbytes(self) -> int:
        """Bytes of the tensor's data: whole blocks, the last one possibly partial."""
        nblocks, rem = divmod(self.numel, self.block_size)
        return (nblocks + (rem > 0)) * self.type_size


@dataclass
class GGUFFile:
    path: Path
    version: int
    metadata: dict[str, GGUFMetadataValue]
    tensors: dict[str, GGUFTensorInfo]
    data_start: int
    alignment: int

    def metadata_value(self, key: str, default: Any = None) -> Any:
        """The decoded value stored under `key`, or `default` when the file has no such key."""
        return self.metadata[key].value if key in self.metadata else default

    def quantized_tensors(self) -> list[GGUFTensorInfo]:
        return list(filter(lambda info: info.is_quantized, self.tensors.values()))

    def mmap_tensor(self, name: str):
        """(file object, mmap, memoryview of the tensor's nbytes bytes). The caller releases the view, then
        closes the mmap and the file."""
        info = self.tensors[name]
        lo, hi = info.absolute_offset, info.absolute_offset + info.nbytes
        fh = self.path.open("rb")
        try:
            mapping = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
            if hi > (size := len(mapping)):
                mapping.close()
                raise UnsupportedModelError(f"tensor {name} ends at byte {hi}, beyond the {size}-byte file")
        except BaseException:
            fh.close()
            raise
        return fh, mapping, memoryview(mapping)[lo:hi]


class _Header:
    """Sequential little-endian reads from the file's start, counting the bytes consumed."""

    def __init__(self, f: BinaryIO) -> None:
        self.f = f
        self.pos = 0

    def take(self, n: int) -> bytes:
        b = self.f.read(n)
        if len(b) != n:
            raise UnsupportedModelError(f"GGUF header ends early: wanted {n} bytes at offset {self.pos}")
        self.pos += n
        return b

    def scalar(self, fmt: str) -> Any:
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        return self.take(self.scalar("<Q")).decode("utf-8")

    def value(self, vt: GGUFValueType) -> Any:
        fmt = _SCALAR_FMT.get(vt)
        if fmt is not None:
            v = self.scalar(fmt)
            return bool(v) if vt is GGUFValueType.BOOL else v
        if vt is GGUFValueType.STRING:
            return self.string()
        if vt is GGUFValueType.ARRAY:
            item = _value_type(self.scalar("<I"))
            return [self.value(item) for _ in range(self.scalar("<Q"))]
        raise UnsupportedModelError(f"metadata values of type {vt.name} cannot be decoded")


def _value_type(raw: int) -> GGUFValueType:
    try:
        return GGUFValueType(raw)
    except ValueError:
        raise UnsupportedModelError(f"metadata value type id {raw} is not defined by GGUF") from None


def load_gguf(path: str | Path, *, require_supported_tensors: bool = False) -> GGUFFile:
    """Parse the header of a GGUF v2/v3 file (load_gguf, parser.py:162-167). With require_supported_tensors,
    every tensor type must have a known block size."""
    path = Path(path)
    with path.open("rb") as f:
        h = _Header(f)
        if h.take(4) != GGUF_MAGIC:
            raise UnsupportedModelError(f"{path}: missing GGUF magic")
        version = h.scalar("<I")
        if version not in (2, 3):
            raise UnsupportedModelError(f"{path}: GGUF version {version} is not 2 or 3")
        n_tensors, n_meta = h.scalar("<Q"), h.scalar("<Q")
        metadata: dict[str, GGUFMetadataValue] = {}
        for _ in range(n_meta):
            key = h.string()
            vt = _value_type(h.scalar("<I"))
            metadata[key] = GGUFMetadataValue(vt, h.value(vt))
        entries = []
        for _ in range(n_tensors):
            name = h.string()
            dims = tuple(h.scalar("<Q") for _ in range(h.scalar("<I")))
            raw = h.scalar("<I")
            try:
                tt = GGUFTensorType(raw)
            except ValueError:
                raise UnsupportedModelError(f"tensor {name}: type id {raw} is not a GGUF tensor type") from None
            entries.append((name, dims, tt, h.scalar("<Q")))
        header_end = h.pos
    align_item = metadata.get("general.alignment")
    alignment = int(align_item.value) if align_item is not None else DEFAULT_ALIGNMENT
    if alignment <= 0:
        raise UnsupportedModelError(f"{path}: general.alignment = {alignment} (must be > 0)")
    data_start = -(-header_end // alignment) * alignment
    tensors = {name: GGUFTensorInfo(name, dims, tt, rel, data_start + rel) for name, dims, tt, rel in entries}
    out = GGUFFile(path, version, metadata, tensors, data_start, alignment)
    if require_supported_tensors:
        for t in tensors.values():
            if t.tensor_type not in GGUF_TYPE_TRAITS:
                raise UnsupportedModelError(f"tensor {t.name}: no block size known for {t.tensor_type.name}")
    return out
