"""Backward of the fused int8 prologues (drop-in for ``int8_backward.py``).

Same functions, arguments and results as the reference (``int8_backward.py:7-89``):
``rmsnorm_backward(grad_y, x, w, eps) -> (grad_x, grad_w)`` and
``gelu_backward(grad_y, x) -> grad_x``. grad_x is rounded to bf16 and stored in x's
dtype (``int8_backward.py:27, 74``); grad_w is summed in float32 and returned in w's
dtype (``int8_backward.py:45-51``). Both run as gfx950 HIP kernels
(``rk_rmsnorm_backward`` / ``rk_gelu_backward``). RMSNorm rows wider than 4096 columns
run as the same formulas in torch tensor ops on the GPU.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .ops import ratchet as _ops

_SQRT_2_OVER_PI = 0.7978845608028654
_MAX_NORM_K = 4096


def _rows(t: Tensor) -> Tensor:
    """[..., K] -> [M, K] with unit column stride (a view when possible)."""
    flat = t.reshape(-1, t.shape[-1])
    if flat.stride(-1) != 1:
        flat = flat.contiguous()
    return flat


def _float_or_bf16(t: Tensor) -> Tensor:
    return t if t.dtype in (torch.float32, torch.bfloat16) else t.float()


def _rmsnorm_backward_torch(gy: Tensor, x_flat: Tensor, w: Tensor, eps: float
                            ) -> tuple[Tensor, Tensor]:
    xf, gf, wf = x_flat.float(), gy.float(), w.float()
    k = xf.shape[1]
    rsqrt = torch.rsqrt((xf * xf).sum(dim=1, keepdim=True) / k + eps)
    dx_hat = gf * wf
    dvar = (dx_hat * xf).sum(dim=1, keepdim=True) * (-0.5) * (rsqrt * rsqrt * rsqrt)
    dx = dx_hat * rsqrt + dvar * 2.0 * xf / k
    return dx.to(torch.bfloat16).to(x_flat.dtype), (gf * xf * rsqrt).sum(dim=0)


def rmsnorm_backward(grad_y: Tensor, x: Tensor, w: Tensor, eps: float = 1e-5, *,
                     residual_grad: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """``residual_grad`` (float32 x only): the gradient x also receives as the residual
    stream, added to grad_x in the same pass (the float32 add autograd would do)."""
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    x_flat = _rows(_float_or_bf16(x))
    gy = _rows(_float_or_bf16(grad_y))
    m, k = x_flat.shape
    if gy.shape != x_flat.shape:
        raise ValueError(f"grad_y {tuple(grad_y.shape)} does not match x {tuple(x.shape)}")
    wf = w.float().contiguous()
    fuse = residual_grad is not None and x_flat.dtype == torch.float32 and k <= _MAX_NORM_K \
        and residual_grad.dtype == torch.float32
    if k > _MAX_NORM_K:
        grad_x, grad_w = _rmsnorm_backward_torch(gy, x_flat, wf, eps)
    elif fuse:
        grad_x, grad_w = _ops().rmsnorm_backward(gy, x_flat, wf, float(eps),
                                                 _rows(residual_grad))
    else:
        grad_x, grad_w = _ops().rmsnorm_backward(gy, x_flat, wf, float(eps))
    grad_x = grad_x.to(x.dtype).reshape(x.shape)
    if residual_grad is not None and not fuse:
        grad_x = grad_x + residual_grad
    return grad_x, grad_w.to(w.dtype)


def gelu_backward(grad_y: Tensor, x: Tensor) -> Tensor:
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    x_flat = _rows(_float_or_bf16(x))
    gy = _rows(_float_or_bf16(grad_y))
    if gy.shape != x_flat.shape:
        raise ValueError(f"grad_y {tuple(grad_y.shape)} does not match x {tuple(x.shape)}")
    grad_x = _ops().gelu_backward(gy, x_flat)
    return grad_x.to(x.dtype).reshape(x.shape)
