"""IQ codebooks expanded on the host from csrc/vq_iq_grids.h (ggml data, MIT licence).

table(name) returns the same byte layout as the reference's tables (entry i at [width*i, width*(i+1)),
byte j = magnitude j): iq2xxs_grid, iq2xs_grid, iq2s_grid (8 bytes per entry), iq3xxs_grid and
iq3s_grid (4 bytes per entry), ksigns_iq2xs (128 bytes).
"""
from __future__ import annotations

import functools
import re
from pathlib import Path

_HEADER = Path(__file__).resolve().parent / "csrc" / "vq_iq_grids.h"
_IQ2_LEVELS = (8, 25, 43)
_IQ3XXS_LEVELS = (4, 12, 20, 28, 36, 44, 52, 62)


@functools.lru_cache(maxsize=None)
def _codes() -> dict[str, list[int]]:
    text = _HEADER.read_text()
    out = {}
    for m in re.finditer(r"uint16_t (\w+)\[(\d+)\] = \{(.*?)\};", text, re.S):
        vals = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", m.group(3))]
        assert len(vals) == int(m.group(2))
        out[m.group(1)] = vals
    return out


@functools.lru_cache(maxsize=None)
def table(name: str) -> bytes:
    c = _codes()
    if name in ("iq2xxs_grid", "iq2xs_grid", "iq2s_grid"):
        key = "vq_" + name.replace("_grid", "_codes")
        return bytes(_IQ2_LEVELS[(code >> (2 * j)) & 3] for code in c[key] for j in range(8))
    if name == "iq3xxs_grid":
        return bytes(_IQ3XXS_LEVELS[(code >> (3 * j)) & 7] for code in c["vq_iq3xxs_codes"] for j in range(4))
    if name == "iq3s_grid":
        return bytes(2 * ((code >> (3 * j)) & 7) + 1 for code in c["vq_iq3s_codes"] for j in range(4))
    if name == "ksigns_iq2xs":
        return bytes(i | ((bin(i).count("1") & 1) << 7) for i in range(128))
    raise KeyError(name)
