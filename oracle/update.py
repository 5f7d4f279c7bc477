"""Integer ratchet update and row normalization (test infrastructure only).

Packed state (``ratchet.py:185-199``): one uint8 per weight,
low nibble = code + max_code, high nibble = pressure + 7.

Update (``ratchet.py:248-301``), all integer given the normalized gradient z:

    inc  = -sign(z) * (|z| >= high ? 2 : |z| >= low ? 1 : 0)
    p'   = p + inc                          (int16)
    PR   = p' >= T,   NR = p' <= -T
    PM   = PR and c <  max_code,   NM = NR and c > -max_code
    c'   = c + PM - NM
    p''  = clamp(p' - PR*T + NR*T, -128, 127)
    byte = ((c' + max_code) & 15) | (((p'' + 7) & 15) << 4)
    counts = (sum PM, sum NM, sum PR & !PM, sum NR & !NM)

Normalization (``ratchet.py:539-556``): z = g / (sqrt(mean_k g^2) + eps), or with the
opt-in per-row EMA of the mean square. The mean square here uses the HIP kernel's fixed
reduction order (``lane_order_sum``) so that the HIP kernel is reproducible bit for bit;
the reference's own order (a BLAS/ATen reduction) is not reproducible by any other
implementation.
"""

from __future__ import annotations

import numpy as np

LANES = 64


def pack(code: np.ndarray, pressure: np.ndarray, max_code: int) -> np.ndarray:
    low = (np.asarray(code, dtype=np.int16) + max_code) & 0x0F
    high = (np.asarray(pressure, dtype=np.int16) + 7) & 0x0F
    return (low | (high << 4)).astype(np.uint8)


def unpack(packed: np.ndarray, max_code: int):
    v = np.asarray(packed, dtype=np.int16)
    code = ((v & 0x0F) - max_code).astype(np.int8)
    pressure = ((v >> 4) - 7).astype(np.int8)
    return code, pressure


def bucket_pressure(z: np.ndarray, low: float = 0.5, high: float = 1.5) -> np.ndarray:
    if not 0 <= low < high:
        raise ValueError("pressure bucket thresholds must satisfy 0 <= low < high")
    z = np.asarray(z, dtype=np.float32)
    mag = np.abs(z)
    bucket = np.where(mag >= np.float32(high), 2, np.where(mag >= np.float32(low), 1, 0))
    sign = np.where(z > 0, 1, np.where(z < 0, -1, 0))  # NaN -> 0
    return (-sign * bucket).astype(np.int16)


def update_core(packed: np.ndarray, z: np.ndarray, max_code: int, threshold: int,
                low: float = 0.5, high: float = 1.5):
    """Returns (new_packed uint8, counts int64[4]) for a normalized gradient z."""
    inc = bucket_pressure(z, low, high).astype(np.int32)
    code, pressure = unpack(packed, max_code)
    c = code.astype(np.int32)
    p = pressure.astype(np.int32) + inc
    pr = p >= threshold
    nr = p <= -threshold
    pm = pr & (c < max_code)
    nm = nr & (c > -max_code)
    c = c + pm.astype(np.int32) - nm.astype(np.int32)
    p = p - pr.astype(np.int32) * threshold + nr.astype(np.int32) * threshold
    p = np.clip(p, -128, 127)
    new = (((c + max_code) & 0x0F) | (((p + 7) & 0x0F) << 4)).astype(np.uint8)
    counts = np.array([pm.sum(), nm.sum(), (pr & ~pm).sum(), (nr & ~nm).sum()], dtype=np.int64)
    return new, counts


def vec_for_dtype(dtype: str) -> int:
    """Elements per lane chunk: one 16-byte vector of the gradient dtype."""
    return {"f32": 4, "bf16": 8}[dtype]


def lane_order_sum(terms: np.ndarray, vec: int) -> np.ndarray:
    """Row sums of float32 ``terms`` [R, K] in the HIP kernels' fixed order.

    One 64-lane wavefront per row. Element e belongs to chunk c = e // (64*vec),
    lane l = (e % (64*vec)) // vec, slot v = e % vec. Each lane accumulates
    acc = acc + term over (c ascending, v ascending) with separately rounded fp32
    adds; the 64 lane totals are then combined by an xor butterfly
    (offsets 32, 16, 8, 4, 2, 1; acc = acc + acc[lane ^ offset]).
    """
    terms = np.asarray(terms, dtype=np.float32)
    rows, k = terms.shape
    span = LANES * vec
    chunks = max(1, -(-k // span))
    padded = np.zeros((rows, chunks * span), dtype=np.float32)
    padded[:, :k] = terms
    x = padded.reshape(rows, chunks, LANES, vec)
    acc = np.zeros((rows, LANES), dtype=np.float32)
    for c in range(chunks):
        for v in range(vec):
            acc = acc + x[:, c, :, v]
    lanes = np.arange(LANES)
    for off in (32, 16, 8, 4, 2, 1):
        acc = acc + acc[:, lanes ^ off]
    return acc[:, 0].copy()


def row_sumsq(g: np.ndarray, vec: int) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    return lane_order_sum(g * g, vec)


def normalize_rows(g: np.ndarray, eps: float, vec: int, rms_ema: np.ndarray | None = None,
                   beta: float = 0.0):
    """Returns (z, instantaneous row rms, new rms_ema or None)."""
    g = np.asarray(g, dtype=np.float32)
    k = g.shape[1]
    ms = row_sumsq(g, vec) / np.float32(k)
    rms_inst = np.sqrt(ms).astype(np.float32)
    ema_new = None
    if rms_ema is not None:
        ema = np.asarray(rms_ema, dtype=np.float32)
        b1 = np.float32(beta)
        b2 = np.float32(1.0 - beta)
        upd = np.where(ema == 0, ms, (b1 * ema + b2 * ms).astype(np.float32))
        ema_new = np.where(ms > 0, upd, ema).astype(np.float32)
        rms = np.sqrt(ema_new).astype(np.float32)
    else:
        rms = rms_inst
    d = (rms + np.float32(eps)).astype(np.float32)
    z = (g / d[:, None]).astype(np.float32)
    return z, rms_inst, ema_new


def update_from_gradient(packed: np.ndarray, g: np.ndarray, max_code: int, threshold: int,
                         low: float, high: float, eps: float, vec: int,
                         rms_ema: np.ndarray | None = None, beta: float = 0.0):
    """Fused normalize + update over whole rows.

    Rows holding a NaN/Inf are left unchanged and reported through ``nonfinite``.
    Returns dict(packed, counts, row_rms, rms_ema, nonfinite, grad_scale).
    """
    packed = np.asarray(packed, dtype=np.uint8)
    g = np.asarray(g, dtype=np.float32)
    finite_rows = np.isfinite(g).all(axis=1)
    z, rms_inst, ema_new = normalize_rows(g, eps, vec, rms_ema, beta)
    new, _ = update_core(packed, z, max_code, threshold, low, high)
    new = np.where(finite_rows[:, None], new, packed)
    counts = np.zeros(4, dtype=np.int64)
    if finite_rows.any():
        _, counts = update_core(packed[finite_rows], z[finite_rows], max_code, threshold,
                                low, high)
    if ema_new is not None:
        ema_new = np.where(finite_rows, ema_new, rms_ema)
    code, _ = unpack(packed, max_code)
    grad_scale = lane_order_sum(g * code.astype(np.float32), vec)
    return {
        "packed": new,
        "counts": counts,
        "row_rms": rms_inst,
        "rms_ema": ema_new,
        "nonfinite": int((~finite_rows).any()),
        "grad_scale": grad_scale,
    }


def pressure_leak(packed: np.ndarray, max_code: int) -> np.ndarray:
    """Move every nonzero pressure one unit toward zero (``ratchet.py:613-625``)."""
    code, pressure = unpack(packed, max_code)
    p = pressure.astype(np.int16)
    return pack(code, p - np.sign(p), max_code)
