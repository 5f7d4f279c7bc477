"""The reference's CPU path for one ratchet linear, restated in eager torch (CPU baseline).

Test / baseline infrastructure only. The reference's int8 path is GPU-only
(``int8_matmul.py:257-258``); its CPU path is ``matmul_mode="fp32"`` with the update
fused into backward over 256-row tiles. One step here is that path:

* forward  ``out = x @ (code * scale)^T``                      (ratchet.py:57-59)
* backward ``grad_input = g @ (code * scale)``                 (ratchet.py:120-124)
* per 256-row tile: ``G_w = g[:, tile]^T @ x``,
  ``z = G_w / (sqrt(mean G_w^2) + eps)``, integer update      (ratchet.py:150-169,
  539-556, 265-301)

It is timed on the host cores as the ``cpu_baseline`` of bench.py, in the same unit
(TOPS over the three GEMMs' 2*M*N*K each) as the GPU path.
"""

from __future__ import annotations

import torch


def _update_core(packed, z, max_code, threshold, low, high):
    mag = z.abs()
    inc = -torch.sign(z).to(torch.int16) * ((mag >= high).to(torch.int16)
                                            + (mag >= low).to(torch.int16))
    v = packed.to(torch.int16)
    code = (v & 0x0F) - max_code
    p = (v >> 4) - 7 + inc
    pr = p >= threshold
    nr = p <= -threshold
    pm = pr & (code < max_code)
    nm = nr & (code > -max_code)
    code = code + pm.to(torch.int16) - nm.to(torch.int16)
    p = (p - pr.to(torch.int16) * threshold + nr.to(torch.int16) * threshold).clamp(-128, 127)
    new = ((code + max_code) & 0x0F) | (((p + 7) & 0x0F) << 4)
    return new.to(torch.uint8), pm.sum() + nm.sum()


def fp32_ratchet_linear_step(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor,
                             grad_out: torch.Tensor, max_code: int, threshold: int = 8,
                             low: float = 0.5, high: float = 1.5, eps: float = 1e-8,
                             tile_size: int = 256):
    """One fp32 forward + backward + fused update; mutates ``packed``. Returns
    (output, grad_input, code_moves)."""
    code = ((packed.to(torch.int16) & 0x0F) - max_code).to(torch.float32)
    effective = code * scale[:, None]
    out = x @ effective.t()
    grad_input = grad_out @ effective
    moves = torch.zeros((), dtype=torch.int64)
    grad_t = grad_out.t()
    for t0 in range(0, packed.shape[0], tile_size):
        t1 = min(t0 + tile_size, packed.shape[0])
        gw = grad_t[t0:t1] @ x
        rms = gw.square().mean(dim=1, keepdim=True).sqrt()
        z = gw / (rms + eps)
        new, m = _update_core(packed[t0:t1], z, max_code, threshold, low, high)
        packed[t0:t1] = new
        moves += m
    return out, grad_input, moves
