"""Bit-exact bfloat16 / float16 rounding on numpy arrays (test infrastructure only).

numpy has no bfloat16, so values are carried as float32 arrays that hold exactly
representable bf16 numbers, or as uint16 bit patterns.  Rounding is IEEE
round-to-nearest-even, which is what torch's ``.to(torch.bfloat16)`` does.

Pinned by ``tests/test_oracle_w3.py::test_bf16_rounding_matches_torch`` against
torch's own conversion on every float32 exponent and on ties.
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(values) -> np.ndarray:
    """Round float32 values to bf16 (nearest-even); return uint16 bit patterns."""
    f = np.ascontiguousarray(values, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    if nan.any():
        out = np.where(nan, np.uint16(0x7FC0), out)
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(values) -> np.ndarray:
    """float32 -> nearest bf16, returned as float32 holding the bf16 value."""
    return bf16_bits_to_f32(f32_to_bf16_bits(values))


def round_f16(values) -> np.ndarray:
    """float32 -> nearest float16, returned as float32."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(values, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` in {"f32", "f16", "bf16"}; float32 result."""
    if dtype == "bf16":
        return round_bf16(values)
    if dtype == "f16":
        return round_f16(values)
    if dtype == "f32":
        return np.asarray(values, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype}")
