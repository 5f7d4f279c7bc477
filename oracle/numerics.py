"""Bit-level float helpers shared by the oracle modules (test infrastructure only).

bf16 conversion follows round-to-nearest-even with NaN mapped to 0x7FC0, which is
what ``torch.Tensor.to(torch.bfloat16)`` does (c10 ``round_to_nearest_even``) and
therefore what the reference's ``.to(torch.bfloat16)`` casts produce
(``ratchet.py:73-75``, ``int8_matmul.py:79``).
"""

from __future__ import annotations

import numpy as np

TINY = np.float32(np.finfo(np.float32).tiny)  # torch.finfo(float32).tiny, int8_matmul.py:87


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern (uint16), round-to-nearest-even, NaN -> 0x7FC0."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), rounded).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bit pattern (uint16) -> fp32 (exact widening)."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 values rounded to the nearest bf16, returned as fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
