"""A minimal GGUF v2/v3 writer for the reader's tests (the container layout of vinf_3080ti_amd/gguf.py)."""
from __future__ import annotations

import struct
from pathlib import Path

from vinf_3080ti_amd.gguf import GGUF_MAGIC, GGUFValueType as V

_FMT = {V.UINT8: "<B", V.INT8: "<b", V.UINT16: "<H", V.INT16: "<h", V.UINT32: "<I", V.INT32: "<i",
        V.FLOAT32: "<f", V.BOOL: "<?", V.UINT64: "<Q", V.INT64: "<q", V.FLOAT64: "<d"}


def enc_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def enc_value(vt: V, value) -> bytes:
    if vt in _FMT:
        return struct.pack(_FMT[vt], value)
    if vt is V.STRING:
        return enc_string(value)
    item, items = value  # ARRAY: (item type, list)
    return struct.pack("<IQ", int(item), len(items)) + b"".join(enc_value(item, v) for v in items)


def write_gguf(path: Path, metadata: list[tuple[str, V, object]], tensors: list[tuple[str, tuple[int, ...], int, bytes]],
               *, version: int = 3, alignment: int | None = None, magic: bytes = GGUF_MAGIC) -> list[int]:
    """Write the file; tensors are (name, dims innermost first, type id, payload). Each payload starts at a
    multiple of the alignment inside the data section. Returns the payloads' absolute offsets."""
    align = 32 if alignment is None else alignment
    if alignment is not None:
        metadata = metadata + [("general.alignment", V.UINT32, alignment)]
    rel, off = [], 0
    for _, _, _, payload in tensors:
        rel.append(off)
        off = -(-(off + len(payload)) // align) * align
    head = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(metadata)))
    for key, vt, value in metadata:
        head += enc_string(key) + struct.pack("<I", int(vt)) + enc_value(vt, value)
    for (name, dims, tt, _), r in zip(tensors, rel):
        head += enc_string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", int(tt), r)
    start = -(-len(head) // align) * align
    body = bytearray(off)
    for (_, _, _, payload), r in zip(tensors, rel):
        body[r:r + len(payload)] = payload
    Path(path).write_bytes(bytes(head) + b"\0" * (start - len(head)) + bytes(body))
    return [start + r for r in rel]
