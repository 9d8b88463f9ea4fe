"""GGUF tensor type ids and block traits of the quantized-matvec path.

Mirrors GGUFTensorType / GGUF_TYPE_TRAITS (/root/reference/engine/src/vinf/gguf/parser.py:33-94) for the
types the reference's matvec accepts (CUDA_MATVEC_TYPES, src/vinf/cuda/qwen_runtime.py:10-28).
"""
from __future__ import annotations

from enum import IntEnum


class GGUFTensorType(IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    IQ2_XS = 17
    IQ3_XXS = 18
    IQ1_S = 19
    IQ4_NL = 20
    IQ3_S = 21
    IQ2_S = 22
    IQ4_XS = 23
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    IQ1_M = 29
    BF16 = 30


# (block_size, type_size) for every type this path handles.
TYPE_TRAITS: dict[GGUFTensorType, tuple[int, int]] = {
    GGUFTensorType.F32: (1, 4),
    GGUFTensorType.F16: (1, 2),
    GGUFTensorType.Q8_0: (32, 34),
    GGUFTensorType.Q2_K: (256, 84),
    GGUFTensorType.Q3_K: (256, 110),
    GGUFTensorType.Q4_K: (256, 144),
    GGUFTensorType.Q5_K: (256, 176),
    GGUFTensorType.Q6_K: (256, 210),
    GGUFTensorType.IQ4_NL: (32, 18),
    GGUFTensorType.IQ3_S: (256, 110),
    GGUFTensorType.IQ4_XS: (256, 136),
    GGUFTensorType.IQ2_XXS: (256, 66),
    GGUFTensorType.IQ2_XS: (256, 74),
    GGUFTensorType.IQ2_S: (256, 82),
    GGUFTensorType.IQ3_XXS: (256, 98),
}

# Types with a HIP matvec (the reference's CUDA_MATVEC_TYPES, cuda/qwen_runtime.py:10-28).
HIP_MATVEC_TYPES = frozenset(TYPE_TRAITS)
QUANT_TYPES = tuple(t for t in TYPE_TRAITS if t not in (GGUFTensorType.F32, GGUFTensorType.F16))

# Byte offsets of the fp16 scale fields inside one block (test_phase30_cuda_qmatvec.py:19-33).
F16_FIELDS: dict[GGUFTensorType, tuple[int, ...]] = {
    GGUFTensorType.Q8_0: (0,),
    GGUFTensorType.IQ4_NL: (0,),
    GGUFTensorType.Q4_K: (0, 2),
    GGUFTensorType.Q5_K: (0, 2),
    GGUFTensorType.Q6_K: (208,),
    GGUFTensorType.Q3_K: (108,),
    GGUFTensorType.Q2_K: (80, 82),
    GGUFTensorType.IQ2_XXS: (0,),
    GGUFTensorType.IQ2_XS: (0,),
    GGUFTensorType.IQ2_S: (0,),
    GGUFTensorType.IQ3_XXS: (0,),
    GGUFTensorType.IQ4_XS: (0,),
    GGUFTensorType.IQ3_S: (0,),
}


def traits(tensor_type: int) -> tuple[int, int]:
    try:
        return TYPE_TRAITS[GGUFTensorType(tensor_type)]
    except (ValueError, KeyError):
        raise ValueError(f"unsupported GGUF tensor type id {int(tensor_type)} for HIP matvec") from None


def row_bytes(tensor_type: int, cols: int) -> int:
    bs, ts = traits(tensor_type)
    if cols <= 0 or cols % bs:
        raise ValueError(f"cols={cols} must be a positive multiple of the block size {bs}")
    return cols // bs * ts
