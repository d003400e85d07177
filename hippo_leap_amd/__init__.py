"""hippo_leap_amd: HippoLeap's attention stage, native to MI355X (gfx950).

The compute lives in libhl_attn.so (hand-written HIP kernels behind the C ABI
declared in include/hl_attn.h); this package holds its build script and a
host-side mirror of the reference's Nim attention procs (attention.py).
"""
from ._lib import (HL_BF16, HL_ECAPTURE, HL_EHIP, HL_EINVAL, HL_ECAPACITY, HL_EUNSUPPORTED, HL_F16, HL_F32,
                   HL_OK, HL_ROPE_HALF_SPLIT, HL_ROPE_INTERLEAVED, LIB_PATH, HLError, load)

__all__ = [
    "HL_BF16", "HL_ECAPTURE", "HL_EHIP", "HL_EINVAL", "HL_ECAPACITY", "HL_EUNSUPPORTED", "HL_F16", "HL_F32",
    "HL_OK", "HL_ROPE_HALF_SPLIT", "HL_ROPE_INTERLEAVED", "LIB_PATH", "HLError", "load",
]
