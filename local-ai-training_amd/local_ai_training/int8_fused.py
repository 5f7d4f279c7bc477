"""Fused per-token absmax-quant prologues on gfx950 (drop-in for ``int8_fused.py``).

Each prologue computes its transform and the int8 row quantization in one HIP kernel
(one wavefront per token row): RMSNorm+quant, tanh-GELU+quant and the attention
head-merge transpose+quant (``int8_fused.py:14-151``). The autograd wrappers return
the reference's third "dummy" output so gradient flows through the ratchet layer's
``inputs`` argument (``int8_fused.py:153-201``).
"""

from __future__ import annotations

import torch
from torch import Tensor

from .ops import ratchet as _ops


def _rowwise(x: Tensor) -> Tensor:
    flat = x.flatten(0, -2)
    if flat.dtype not in (torch.float32, torch.bfloat16):
        flat = flat.float()
    return flat


def _dq_rows(x_dq: Tensor | None) -> Tensor | None:
    return None if x_dq is None else x_dq.view(-1, x_dq.shape[-1])


def fused_rmsnorm_quantize(x: Tensor, weight: Tensor, eps: float = 1e-5, *,
                           x_dq: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """``x_dq`` (optional, bf16 of x's shape, contiguous): receives the dequantized rows
    bf16(bf16(q) * bf16(s)) from the same kernel; likewise for the other prologues."""
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    q, scale = _ops().rmsnorm_quantize(_rowwise(x), weight.detach().float(), float(eps),
                                       _dq_rows(x_dq))
    return q.reshape(x.shape), scale.reshape(x.shape[:-1])


def fused_gelu_quantize(x: Tensor, *, x_dq: Tensor | None = None) -> tuple[Tensor, Tensor]:
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    q, scale = _ops().gelu_quantize(_rowwise(x), _dq_rows(x_dq))
    return q.reshape(x.shape), scale.reshape(x.shape[:-1])


def fused_transpose_quantize(x: Tensor, *, x_dq: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """[B, H, S, D] (any strides) -> int8 rows [B*S, H*D] and float32 scales [B*S]
    (``x_dq``: bf16 [B*S, H*D])."""
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    return _ops().transpose_quantize(x, x_dq)


def _new_dq(shape, like: Tensor, dequant: bool) -> Tensor | None:
    return torch.empty(shape, device=like.device, dtype=torch.bfloat16) if dequant else None


def _no_grad_outputs(ctx, int8_out: Tensor, scale_out: Tensor,
                     dq_out: Tensor | None = None) -> None:
    """The int8 values, their scales and the dequantized copy carry no gradient (only the
    dummy output's gradient flows back): mark them so, and do not have autograd build zero
    gradients for outputs nothing used (one fill kernel each per backward otherwise)."""
    ctx.mark_non_differentiable(int8_out, scale_out, *(() if dq_out is None else (dq_out,)))
    ctx.set_materialize_grads(False)


class FusedRMSNormQuantizeFn(torch.autograd.Function):
    """(int8, scale, dummy, dequantized copy or None) of RMSNorm(x) * weight; ``dequant``
    asks for the bf16 dequantized copy (the ratchet layer's backward operand)."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, eps: float = 1e-5, dequant: bool = False):
        dq = _new_dq(x.shape, x, dequant)
        int8_out, scale_out = fused_rmsnorm_quantize(x, weight, eps, x_dq=dq)
        ctx.save_for_backward(x, weight)
        ctx.eps = eps
        _no_grad_outputs(ctx, int8_out, scale_out, dq)
        return int8_out, scale_out, torch.empty_like(x), dq

    @staticmethod
    def backward(ctx, grad_int8, grad_scale, grad_dummy, grad_dq):
        if grad_dummy is None:
            return None, None, None, None
        x, weight = ctx.saved_tensors
        from .int8_backward import rmsnorm_backward

        grad_x, grad_w = rmsnorm_backward(grad_dummy, x, weight, ctx.eps)
        return grad_x, grad_w, None, None


class FusedRMSNormQuantizeResidualFn(torch.autograd.Function):
    """FusedRMSNormQuantizeFn for an x that also continues as the residual stream: returns
    (int8, scale, dummy, x, dequantized copy or None). Both of x's gradients then arrive in this backward, which adds
    them in the RMSNorm backward kernel's store (the same float32 add autograd performs when
    x feeds two separate uses) instead of a separate add kernel."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, eps: float = 1e-5, dequant: bool = False):
        dq = _new_dq(x.shape, x, dequant)
        int8_out, scale_out = fused_rmsnorm_quantize(x, weight, eps, x_dq=dq)
        ctx.save_for_backward(x, weight)
        ctx.eps = eps
        _no_grad_outputs(ctx, int8_out, scale_out, dq)
        return int8_out, scale_out, torch.empty_like(x), x.view_as(x), dq

    @staticmethod
    def backward(ctx, grad_int8, grad_scale, grad_dummy, grad_residual, grad_dq):
        x, weight = ctx.saved_tensors
        if grad_dummy is None:
            return grad_residual, None, None, None
        from .int8_backward import rmsnorm_backward

        grad_x, grad_w = rmsnorm_backward(grad_dummy, x, weight, ctx.eps,
                                          residual_grad=grad_residual)
        return grad_x, grad_w, None, None


class FusedGELUQuantizeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: Tensor, dequant: bool = False):
        dq = _new_dq(x.shape, x, dequant)
        int8_out, scale_out = fused_gelu_quantize(x, x_dq=dq)
        ctx.save_for_backward(x)
        _no_grad_outputs(ctx, int8_out, scale_out, dq)
        return int8_out, scale_out, torch.empty_like(x), dq

    @staticmethod
    def backward(ctx, grad_int8, grad_scale, grad_dummy, grad_dq):
        if grad_dummy is None:
            return None, None
        (x,) = ctx.saved_tensors
        from .int8_backward import gelu_backward

        return gelu_backward(grad_dummy, x), None


class FusedTransposeQuantizeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, attended: Tensor, dequant: bool = False):
        batch_size, n_head, seq_len, head_dim = attended.shape
        dq = _new_dq((batch_size * seq_len, n_head * head_dim), attended, dequant)
        int8_out, scale_out = fused_transpose_quantize(attended, x_dq=dq)
        ctx.shape = attended.shape
        dummy = torch.empty((batch_size, seq_len, n_head * head_dim), device=attended.device,
                            dtype=attended.dtype)
        _no_grad_outputs(ctx, int8_out, scale_out, dq)
        return int8_out, scale_out, dummy, dq

    @staticmethod
    def backward(ctx, grad_int8, grad_scale, grad_dummy, grad_dq):
        if grad_dummy is None:
            return None, None
        batch_size, n_head, seq_len, head_dim = ctx.shape
        return grad_dummy.view(batch_size, seq_len, n_head, head_dim).transpose(1, 2), None
