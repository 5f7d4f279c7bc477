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


def fused_rmsnorm_quantize(x: Tensor, weight: Tensor, eps: float = 1e-5) -> tuple[Tensor, Tensor]:
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    q, scale = _ops().rmsnorm_quantize(_rowwise(x), weight.detach().float(), float(eps))
    return q.reshape(x.shape), scale.reshape(x.shape[:-1])


def fused_gelu_quantize(x: Tensor) -> tuple[Tensor, Tensor]:
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    q, scale = _ops().gelu_quantize(_rowwise(x))
    return q.reshape(x.shape), scale.reshape(x.shape[:-1])


def fused_transpose_quantize(x: Tensor) -> tuple[Tensor, Tensor]:
    """[B, H, S, D] (any strides) -> int8 rows [B*S, H*D] and float32 scales [B*S]."""
    if not x.is_cuda:
        raise RuntimeError("CUDA required (a ROCm GPU)")
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    return _ops().transpose_quantize(x)


def _no_grad_outputs(ctx, int8_out: Tensor, scale_out: Tensor) -> None:
    """The int8 values and their scales carry no gradient (only the dummy output's gradient
    flows back): mark them so, and do not have autograd build zero gradients for outputs
    nothing used (one fill kernel each per backward otherwise)."""
    ctx.mark_non_differentiable(int8_out, scale_out)
    ctx.set_materialize_grads(False)


class FusedRMSNormQuantizeFn(torch.autograd.Function):
    """(int8, scale, dummy) of RMSNorm(x) * weight (int8_fused.py:153-167)."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, eps: float = 1e-5):
        int8_out, scale_out = fused_rmsnorm_quantize(x, weight, eps)
        ctx.save_for_backward(x, weight)
        ctx.eps = eps
        _no_grad_outputs(ctx, int8_out, scale_out)
        return int8_out, scale_out, torch.empty_like(x)

    @staticmethod
    def backward(ctx, grad_int8, grad_scale, grad_dummy):
        if grad_dummy is None:
            return None, None, None
        x, weight = ctx.saved_tensors
        from .int8_backward import rmsnorm_backward

        grad_x, grad_w = rmsnorm_backward(grad_dummy, x, weight, ctx.eps)
        return grad_x, grad_w, None


class FusedRMSNormQuantizeResidualFn(torch.autograd.Function):
    """FusedRMSNormQuantizeFn for an x that also continues as the residual stream: returns
    (int8, scale, dummy, x). Both of x's gradients then arrive in this backward, which adds
    them in the RMSNorm backward kernel's store (the same float32 add autograd performs when
    x feeds two separate uses) instead of a separate add kernel."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, eps: float = 1e-5):
        int8_out, scale_out = fused_rmsnorm_quantize(x, weight, eps)
        ctx.save_for_backward(x, weight)
        ctx.eps = eps
        _no_grad_outputs(ctx, int8_out, scale_out)
        return int8_out, scale_out, torch.empty_like(x), x.view_as(x)

    @staticmethod
    def backward(ctx, grad_int8, grad_scale, grad_dummy, grad_residual):
        x, weight = ctx.saved_tensors
        if grad_dummy is None:
            return grad_residual, None, None
        from .int8_backward import rmsnorm_backward

        grad_x, grad_w = rmsnorm_backward(grad_dummy, x, weight, ctx.eps,
                                          residual_grad=grad_residual)
        return grad_x, grad_w, None


class FusedGELUQuantizeFn(torch.autograd.Function):
    """(int8, scale, dummy) of tanh-GELU(x) (int8_fused.py:169-182)."""

    @staticmethod
    def forward(ctx, x: Tensor):
        int8_out, scale_out = fused_gelu_quantize(x)
        ctx.save_for_backward(x)
        _no_grad_outputs(ctx, int8_out, scale_out)
        return int8_out, scale_out, torch.empty_like(x)

    @staticmethod
    def backward(ctx, grad_int8, grad_scale, grad_dummy):
        if grad_dummy is None:
            return None
        (x,) = ctx.saved_tensors
        from .int8_backward import gelu_backward

        return gelu_backward(grad_dummy, x)


class FusedTransposeQuantizeFn(torch.autograd.Function):
    """(int8, scale, dummy) of the attention head merge (int8_fused.py:184-201)."""

    @staticmethod
    def forward(ctx, attended: Tensor):
        batch_size, n_head, seq_len, head_dim = attended.shape
        int8_out, scale_out = fused_transpose_quantize(attended)
        ctx.shape = attended.shape
        dummy = torch.empty((batch_size, seq_len, n_head * head_dim), device=attended.device,
                            dtype=attended.dtype)
        _no_grad_outputs(ctx, int8_out, scale_out)
        return int8_out, scale_out, dummy

    @staticmethod
    def backward(ctx, grad_int8, grad_scale, grad_dummy):
        if grad_dummy is None:
            return None
        batch_size, n_head, seq_len, head_dim = ctx.shape
        return grad_dummy.view(batch_size, seq_len, n_head, head_dim).transpose(1, 2)
