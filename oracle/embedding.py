"""Token-embedding weight gradient — TEST INFRASTRUCTURE ONLY (CPU oracle).

The reference's model looks tokens up in an ``nn.Embedding`` (``model.py:219``, used at
``model.py:237``); its backward gives each vocabulary row the sum of the gradient rows of
the tokens with that id. The HIP kernels (``rk_embedding_backward``) fix the float32
summation order: tokens in chunks of ``CHUNK`` consecutive positions, token order within a
chunk, then the per-chunk sums in chunk order. This restates that order exactly.

Pinning: on integer-valued gradients every partial sum is exact, so any order gives the
same bits; there the result equals torch's own embedding backward on the CPU (the
reference's op) bit for bit. On general floats it agrees with torch's within float32
reassociation error.
"""

from __future__ import annotations

import numpy as np

CHUNK = 64


def embedding_backward(grad: np.ndarray, ids: np.ndarray, num_weights: int,
                       chunk: int = CHUNK) -> np.ndarray:
    """float32 [num_weights, D]: row v = sum over tokens t with ids[t] == v of grad[t], in the
    chunked order above; ids outside [0, num_weights) contribute nothing."""
    g = np.ascontiguousarray(grad, dtype=np.float32).reshape(-1, grad.shape[-1])
    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    if flat.shape[0] != g.shape[0]:
        raise ValueError("one gradient row per id")
    out = np.zeros((num_weights, g.shape[1]), dtype=np.float32)
    for c0 in range(0, flat.shape[0], chunk):
        part: dict[int, np.ndarray] = {}
        for t in range(c0, min(c0 + chunk, flat.shape[0])):
            v = int(flat[t])
            if not 0 <= v < num_weights:
                continue
            part[v] = g[t].copy() if v not in part else (part[v] + g[t]).astype(np.float32)
        for v, p in part.items():
            out[v] = (out[v] + p).astype(np.float32)
    return out
