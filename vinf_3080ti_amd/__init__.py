"""MI355X-native (gfx950) GGUF quantized-weight matvec hot path of the vinf engine.

Public surface:
  Runtime, HipWeightRuntime   name-keyed device runtime mirroring vinf's CUDA runtime on this path
  GGUFTensorType, TYPE_TRAITS GGUF type ids and block traits
  synth                       seeded synthetic GGUF weights
The compute lives in libvq_hip.so (C ABI: include/vq.h); there is no CPU fallback.
"""
from .gguf_types import GGUFTensorType, HIP_MATVEC_TYPES, QUANT_TYPES, TYPE_TRAITS, row_bytes, traits

__all__ = ["GGUFTensorType", "HIP_MATVEC_TYPES", "QUANT_TYPES", "TYPE_TRAITS", "row_bytes", "traits",
           "Runtime", "HipWeightRuntime"]


def __getattr__(name):
    if name in ("Runtime", "HipWeightRuntime"):
        from . import runtime

        return getattr(runtime, name)
    raise AttributeError(name)
