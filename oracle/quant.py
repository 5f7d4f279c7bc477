"""Per-token absmax int8 quantization, deterministic and stochastic (test infrastructure only).

Follows ``int8_matmul.py:106-150`` (``_quantize_rows_kernel``) and its torch oracle
``int8_matmul.py:225-239`` (``_quantize_rows_reference``):

    x     = float32(v)                         (optionally * col_scale[k], one fp32 multiply)
    amax  = max_k |x|
    scale = max(amax / 127, FLT_MIN)           (IEEE fp32 division)
    det:  q = clamp(roundTiesToEven(x / scale), -127, 127)
    SR:   q = clamp(floor(x / scale + u), -127, 127),  u = rand(seed, m * K + k)

Inputs are float32 arrays; a bf16 input is passed already widened (exact).
"""

from __future__ import annotations

import numpy as np

from .numerics import TINY
from .philox import rand, sr_offsets

_D127 = np.float32(127.0)


def _prepared(values: np.ndarray, col_scale: np.ndarray | None) -> np.ndarray:
    x = np.asarray(values, dtype=np.float32)
    if x.ndim != 2:
        raise ValueError("row quantization requires a 2D tensor")
    if col_scale is not None:
        x = x * np.asarray(col_scale, dtype=np.float32)[None, :]
    return x


def row_scale(x: np.ndarray) -> np.ndarray:
    amax = np.abs(x).max(axis=1) if x.shape[1] else np.zeros(x.shape[0], np.float32)
    return np.maximum(amax.astype(np.float32) / _D127, TINY).astype(np.float32)


def quantize_rows(values: np.ndarray, col_scale: np.ndarray | None = None):
    """Deterministic row quantization; returns (int8 [M,K], float32 [M])."""
    x = _prepared(values, col_scale)
    scale = row_scale(x)
    y = x / scale[:, None]
    q = np.clip(np.rint(y), -127.0, 127.0).astype(np.int8)
    return q, scale


def quantize_rows_sr(values: np.ndarray, col_scale: np.ndarray | None, seed: int,
                     row_start: int = 0):
    """Stochastic row quantization with Philox bits; returns (int8 [M,K], float32 [M]).

    ``row_start`` offsets the row index inside the counter (m is the global row).
    """
    x = _prepared(values, col_scale)
    scale = row_scale(x)
    y = x / scale[:, None]
    u = rand(seed, sr_offsets(x.shape[0], x.shape[1], row_start))
    r = np.floor((y + u).astype(np.float32))
    q = np.clip(r, -127.0, 127.0).astype(np.int8)
    return q, scale


def quantize_columns(values: np.ndarray):
    """Per-column absmax quantization (``int8_matmul.py:242-248``)."""
    q, s = quantize_rows(np.asarray(values, dtype=np.float32).T)
    return np.ascontiguousarray(q.T), s
