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


# float16 (IEEE half) counterparts, for the float16 form of the fused linear
# (the reference's X_DTYPE / LORA_DTYPE = float16, lora_forward.py:141-143).
# numpy's float32 -> float16 conversion rounds to nearest even, as torch's
# ``.to(torch.float16)`` and tl.cast do.

def f32_to_f16_bits(x) -> np.ndarray:
    """Round float32 values to float16 (RNE); returns uint16 bit patterns."""
    with np.errstate(over="ignore"):  # beyond float16's range: inf, as the cast gives
        h = np.asarray(x, dtype=np.float32).astype(np.float16)
    return np.ascontiguousarray(h).view(np.uint16)


def f16_bits_to_f32(b) -> np.ndarray:
    """Widen float16 bit patterns (uint16) to float32 exactly."""
    return np.ascontiguousarray(np.asarray(b, dtype=np.uint16)).view(np.float16).astype(np.float32)


def round_f16(x) -> np.ndarray:
    """float32 -> float16 (RNE) -> float32."""
    return f16_bits_to_f32(f32_to_f16_bits(x))


def to_bits(x, dtype: str = "bf16") -> np.ndarray:
    """Round float32 to ``dtype`` ("bf16" or "f16"); uint16 bit patterns."""
    return f32_to_f16_bits(x) if dtype == "f16" else f32_to_bf16_bits(x)


def from_bits(b, dtype: str = "bf16") -> np.ndarray:
    """``dtype`` bit patterns to float32 (exact)."""
    return f16_bits_to_f32(b) if dtype == "f16" else bf16_bits_to_f32(b)


def round_to(x, dtype: str = "bf16") -> np.ndarray:
    """float32 -> ``dtype`` (RNE) -> float32."""
    return round_f16(x) if dtype == "f16" else round_bf16(x)
