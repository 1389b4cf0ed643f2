"""bfloat16 helpers for the oracle (test infrastructure only).

bfloat16 values are carried as ``uint16`` bit patterns so that every rounding
point is explicit.  Rounding is IEEE round-to-nearest-even, which is what the
reference's ``tl.cast(x, tl.bfloat16)`` (``lora_forward.py:206, 243, 246, 253``)
and torch's ``.to(torch.bfloat16)`` do.
"""

from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round float32 values to bfloat16 (RNE); returns uint16 bit patterns."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_bits_to_f32(b) -> np.ndarray:
    """Widen bfloat16 bit patterns (uint16) to float32 exactly."""
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """float32 -> bfloat16 (RNE) -> float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
