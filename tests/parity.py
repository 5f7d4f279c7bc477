"""Oracle checks of one ratchet layer's int8 training step, shared by the layer-shape and
model-level GPU tests.

Each check takes what the GPU produced (and the float producers it consumed) on a set of
rows and replays the integer arithmetic in the numpy oracle:

  forward    out[r] = bf16((q[r] @ code^T) * s[r] * scale)   (+ residual[r], float32 add)
  sr_quant   (gq[r], gs[r]) = SR-quantize(g[r] * scale) with Philox counter (r*N + n)
  grad_input gin[r] = bf16((gq[r] @ code) * gs[r])
  update     packed_after[r] = update(packed_before[r], G_w[r])  (G_w: the bf16 gradient
             the fused update consumed)

Integer outputs, quant scales and bf16 outputs must be identical (bit for bit).
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import gemm as ogemm
from oracle import quant as oquant
from oracle import update as oupd


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.bfloat16).cpu().view(torch.int16).numpy().view(np.uint16)


def f32bits(a) -> np.ndarray:
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def sample_rows(m: int, count: int, seed: int) -> np.ndarray:
    """`count` sorted row indices of [0, m), always including the first and last row."""
    if count >= m:
        return np.arange(m)
    rng = np.random.default_rng(seed)
    inner = rng.choice(np.arange(1, m - 1), size=count - 2, replace=False)
    return np.sort(np.concatenate([[0, m - 1], inner]))


def check_forward(code: np.ndarray, scale: np.ndarray, q: torch.Tensor, s: torch.Tensor,
                  out: torch.Tensor, residual: torch.Tensor | None = None, what: str = "") -> None:
    """q, s, out (and residual) hold the checked rows only; code is [N, K]."""
    want = ogemm.scaled_int8_mm(q.cpu().numpy(), code.T, s.cpu().numpy(), scale)
    if residual is None:
        got = bits16(out) if out.dtype == torch.bfloat16 else None
        if got is None:  # float32 output: the bf16 value widened
            assert np.array_equal(f32bits(out), want.astype(np.uint32) << 16), f"forward {what}"
        else:
            assert np.array_equal(got, want), f"forward {what}"
        return
    widened = (want.astype(np.uint32) << 16).view(np.float32)
    expect = residual.cpu().numpy().astype(np.float32) + widened
    assert np.array_equal(f32bits(out), f32bits(expect)), f"forward+residual {what}"


def check_sr_quant(g: torch.Tensor, scale: np.ndarray, seed: int, rows: np.ndarray,
                   gq: torch.Tensor, gs: torch.Tensor, what: str = "") -> None:
    """g, gq, gs hold the checked rows (global indices `rows`) only."""
    gf = g.float().cpu().numpy()
    gqc, gsc = gq.cpu().numpy(), gs.cpu().numpy()
    # the Philox counter is r * N + n with r the global row: check row runs separately
    starts = np.flatnonzero(np.diff(rows, prepend=-2) != 1)
    for i, start in enumerate(starts):
        end = starts[i + 1] if i + 1 < len(starts) else len(rows)
        q_ref, s_ref = oquant.quantize_rows_sr(gf[start:end], scale, seed,
                                               row_start=int(rows[start]))
        assert np.array_equal(gqc[start:end], q_ref), f"SR quant {what} rows {rows[start]}.."
        assert np.array_equal(f32bits(gsc[start:end]), f32bits(s_ref)), f"SR scale {what}"


def check_grad_input(code: np.ndarray, gq: torch.Tensor, gs: torch.Tensor, gin: torch.Tensor,
                     what: str = "") -> None:
    """gq, gs, gin hold the checked rows only; code is [N, K] (the contraction is over N)."""
    want = ogemm.scaled_int8_mm(gq.cpu().numpy(), code, gs.cpu().numpy(), None)
    if gin.dtype == torch.bfloat16:
        assert np.array_equal(bits16(gin), want), f"grad_input {what}"
    else:
        assert np.array_equal(f32bits(gin), want.astype(np.uint32) << 16), f"grad_input {what}"


def check_update(packed_before: np.ndarray, grad_weight: torch.Tensor, packed_after: np.ndarray,
                 max_code: int, what: str = "", threshold: int = 8, low: float = 0.5,
                 high: float = 1.5, eps: float = 1e-8) -> np.ndarray:
    """Rows of the state before/after and of the consumed bf16 gradient; returns the
    oracle's move counts for those rows."""
    ref = oupd.update_from_gradient(packed_before, grad_weight.float().cpu().numpy(), max_code,
                                    threshold, low, high, eps, oupd.vec_for_dtype("bf16"))
    assert np.array_equal(packed_after, ref["packed"]), f"ratchet state {what}"
    return ref["counts"]
