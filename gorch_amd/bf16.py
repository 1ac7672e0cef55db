"""Host-side bf16 codec, vectorised with numpy: gorch's F32ToBF16Slice and
BF16ToF32Slice (tensor.go:85-121), used to prepare weights for upload.

bf16 values are carried as ``np.uint16`` (the reference's ``data16``).
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even on the low 16 bits; a NaN keeps its top half
    with the quiet bit (0x40) forced (tensor.go:85-94)."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    is_nan = ((bits >> 23) & 0xFF == 0xFF) & ((bits & 0x7FFFFF) != 0)
    rounded = ((bits + (0x7FFF + ((bits >> 16) & 1))) >> 16).astype(np.uint16)
    if is_nan.any():
        rounded = np.where(is_nan, ((bits >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """Exact widening: the 16 bits become the top half of an f32 (tensor.go:97-99)."""
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_f32(x: np.ndarray) -> np.ndarray:
    """f32 values rounded through bf16 (bf16-representable f32)."""
    return bf16_to_f32(f32_to_bf16(x))
