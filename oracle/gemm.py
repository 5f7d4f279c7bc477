"""Scaled int8 GEMM with int32 accumulation and BF16 epilogue (test infrastructure only).

Follows ``int8_matmul.py:26-79`` (``_scaled_int8_kernel``):

    C[m, n] = bf16_RNE( (float32(sum_k A[m,k] * B[k,n]) * ls[m]) * rs[n] )

The integer sum is computed exactly (float64 BLAS on small integers is exact while
|sum| < 2**53; every shape used here is far below 2**24).
"""

from __future__ import annotations

import numpy as np

from .numerics import f32_to_bf16_bits


def int_matmul(lhs: np.ndarray, rhs: np.ndarray) -> np.ndarray:
    """Exact int64 product of int8 matrices [M,K] @ [K,N]."""
    acc = np.asarray(lhs, dtype=np.float64) @ np.asarray(rhs, dtype=np.float64)
    if acc.size and np.abs(acc).max() >= 2.0**53:
        raise OverflowError("accumulator exceeds exact float64 range")
    return acc.astype(np.int64)


def scaled_epilogue(acc: np.ndarray, ls: np.ndarray, rs: np.ndarray | None) -> np.ndarray:
    """fp32 epilogue (acc * ls) * rs, returned as fp32 (before the bf16 rounding)."""
    v = acc.astype(np.float32) * np.asarray(ls, dtype=np.float32)[:, None]
    if rs is not None:
        v = v * np.asarray(rs, dtype=np.float32)[None, :]
    return v.astype(np.float32)


def scaled_int8_mm(lhs: np.ndarray, rhs: np.ndarray, lhs_scale: np.ndarray,
                   rhs_scale: np.ndarray | None) -> np.ndarray:
    """Returns the bf16 bit pattern (uint16 [M,N]) of the scaled product."""
    acc = int_matmul(lhs, rhs)
    return f32_to_bf16_bits(scaled_epilogue(acc, lhs_scale, rhs_scale))
