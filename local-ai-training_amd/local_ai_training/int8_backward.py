"""Backward of the fused int8 prologues (drop-in for ``int8_backward.py``).

The reference computes these in Triton (``int8_backward.py:7-89``) and stores dx
rounded to bf16 into a buffer of the input dtype (``int8_backward.py:27``, ``74``).
They are not part of the ratchet-linear arithmetic; here they are plain tensor
expressions with the same formulas and the same bf16 rounding of dx.
"""

from __future__ import annotations

import torch
from torch import Tensor

_SQRT_2_OVER_PI = 0.7978845608028654


def rmsnorm_backward(grad_y: Tensor, x: Tensor, w: Tensor, eps: float = 1e-5
                     ) -> tuple[Tensor, Tensor]:
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    x_flat = x.flatten(0, -2).float()
    gy = grad_y.flatten(0, -2).float()
    k = x_flat.shape[1]
    wf = w.float()
    variance = (x_flat * x_flat).sum(dim=1, keepdim=True) / k
    rsqrt = torch.rsqrt(variance + eps)
    dx_hat = gy * wf
    dvar = (dx_hat * x_flat).sum(dim=1, keepdim=True) * (-0.5) * (rsqrt * rsqrt * rsqrt)
    dx = dx_hat * rsqrt + dvar * 2.0 * x_flat / k
    grad_x = dx.to(torch.bfloat16).to(x.dtype).reshape(x.shape)
    grad_w = (gy * x_flat * rsqrt).sum(dim=0)
    return grad_x, grad_w.to(w.dtype)


def gelu_backward(grad_y: Tensor, x: Tensor) -> Tensor:
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    xf = x.float()
    gy = grad_y.float()
    x_sq = xf * xf
    t = torch.tanh(_SQRT_2_OVER_PI * (xf + 0.044715 * xf * x_sq))
    term1 = 0.5 * (1.0 + t)
    term2 = 0.5 * xf * (1.0 - t * t) * _SQRT_2_OVER_PI * (1.0 + 0.134145 * x_sq)
    return (gy * (term1 + term2)).to(torch.bfloat16).to(x.dtype)
