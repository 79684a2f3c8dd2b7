"""bf16 bit helpers on the host (numpy), for preparing inputs and reading outputs.

bf16 is stored as the upper 16 bits of an IEEE fp32 (the reference's `BF16 =
type word`, src/quicknn_common.pas:30-31).  Widening is exact (bits << 16,
BF16ToSingle, src/quicknn_common.pas:1991-2008).  Narrowing here rounds to
nearest even, which is what the HIP path applies to fp32 activations; the
reference's own SingleToBF16 truncates (src/quicknn_common.pas:2010-2027).
"""
from __future__ import annotations

import numpy as np


def as_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest, ties to even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    """bf16 bits -> fp32 (exact)."""
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 values rounded to the nearest bf16 value, as fp32."""
    return bf16_bits_to_f32(as_bf16_bits(x))
