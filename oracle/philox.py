"""Counter-based Philox4x32-10 and the uniform map used for stochastic rounding.

Test infrastructure only. Restated from the published algorithm (Salmon, Moraes,
Dror, Shaw, "Parallel Random Numbers: As Easy as 1, 2, 3", SC'11) and from the
call site in the reference: ``int8_matmul.py:143-144`` draws
``u = tl.rand(SEED, m * K + k)``. The reference pins Triton 3.7.1
(``uv.lock:2664-2665``, not vendored); its open-source ``triton/language/random.py``
defines ``rand`` as:

* counter = (offset as uint32, 0, 0, 0) for an int32 offset;
* key     = (seed & 0xffffffff, seed >> 32);
* 10 rounds, round multipliers 0xD2511F53 / 0xCD9E8D57, key increments
  0x9E3779B9 / 0xBB67AE85;
* only the first output word is used;
* word -> float: reinterpret as int32 x, x := (x < 0 ? -x - 1 : x),
  u = float32(x) * float32(4.6566127342e-10)  (so 0 <= u < 1).
"""

from __future__ import annotations

import numpy as np

ROUND_A = np.uint64(0xD2511F53)
ROUND_B = np.uint64(0xCD9E8D57)
KEY_A = np.uint32(0x9E3779B9)
KEY_B = np.uint32(0xBB67AE85)
UNIFORM_SCALE = np.float32(4.6566127342e-10)  # bit pattern 0x2FFFFFFF
_MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32(c0, c1, c2, c3, k0, k1, rounds: int = 10):
    """Philox4x32 bijection on uint32 arrays (broadcasting); returns 4 uint32 arrays."""
    c0 = np.asarray(c0, dtype=np.uint32)
    c1 = np.asarray(c1, dtype=np.uint32)
    c2 = np.asarray(c2, dtype=np.uint32)
    c3 = np.asarray(c3, dtype=np.uint32)
    k0 = np.uint32(k0)
    k1 = np.uint32(k1)
    for _ in range(rounds):
        p0 = ROUND_A * c0.astype(np.uint64)
        p1 = ROUND_B * c2.astype(np.uint64)
        hi0 = (p0 >> np.uint64(32)).astype(np.uint32)
        lo0 = (p0 & _MASK32).astype(np.uint32)
        hi1 = (p1 >> np.uint64(32)).astype(np.uint32)
        lo1 = (p1 & _MASK32).astype(np.uint32)
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        k0 = np.uint32((int(k0) + int(KEY_A)) & 0xFFFFFFFF)
        k1 = np.uint32((int(k1) + int(KEY_B)) & 0xFFFFFFFF)
    return c0, c1, c2, c3


def randint(seed: int, offsets) -> np.ndarray:
    """First Philox output word for counter (offset, 0, 0, 0), key (seed lo, seed hi)."""
    off = np.asarray(offsets, dtype=np.uint32)
    zero = np.zeros_like(off)
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    out, _, _, _ = philox4x32(off, zero, zero, zero, seed & 0xFFFFFFFF, seed >> 32)
    return out


def uint_to_uniform_float(words: np.ndarray) -> np.ndarray:
    """Map uint32 words to float32 in [0, 1) exactly as the Triton 32-bit path does."""
    x = np.asarray(words, dtype=np.uint32).view(np.int32)
    x = np.where(x < 0, ~x, x)  # -x - 1 == ~x in two's complement (no overflow at INT_MIN)
    return x.astype(np.float32) * UNIFORM_SCALE


def rand(seed: int, offsets) -> np.ndarray:
    return uint_to_uniform_float(randint(seed, offsets))


def sr_offsets(rows: int, cols: int, row_start: int = 0) -> np.ndarray:
    """int32 counters m * cols + k (wrapping mod 2**32), ``int8_matmul.py:143``."""
    m = (np.arange(rows, dtype=np.uint64) + np.uint64(row_start))[:, None]
    k = np.arange(cols, dtype=np.uint64)[None, :]
    return ((m * np.uint64(cols) + k) & _MASK32).astype(np.uint32)
