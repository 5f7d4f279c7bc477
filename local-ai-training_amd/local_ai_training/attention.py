"""Causal self-attention of the training step with a HIP forward kernel.

The reference attends with ``F.scaled_dot_product_attention(q, k, v, is_causal=True)``
(``model.py:117-123``). Here the forward is ``rk_attention_forward`` (flash form on the bf16
MFMA, ``csrc/rk_attention.hip``), which writes the output and the per-query log-sum-exp in
the form torch's memory-efficient attention forward does; the backward is torch's own
memory-efficient attention backward, called on those two tensors. torch's forward for this
case ran at 120-210 TFLOP/s on MI355X; the backward is kept as it is.

Supported: bfloat16 GPU q, k, v [B, H, S, D] with D 64 or 128, unit feature stride,
16-byte aligned storage and strides that are multiples of 8 elements, no attention mask,
no dropout, the default scale. Anything else goes to ``F.scaled_dot_product_attention``.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor

from .ops import ratchet

_NO_DROPOUT_SEED: dict[int, tuple[Tensor, Tensor]] = {}


def _philox_placeholders() -> tuple[Tensor, Tensor]:
    """The (seed, offset) pair the memory-efficient backward takes; unused without dropout."""
    key = 0
    if key not in _NO_DROPOUT_SEED:
        _NO_DROPOUT_SEED[key] = (torch.zeros((), dtype=torch.int64),
                                 torch.zeros((), dtype=torch.int64))
    return _NO_DROPOUT_SEED[key]


def _extent_fits(shape: tuple[int, ...], stride: tuple[int, ...]) -> bool:
    """The kernel's 32-bit buffer offsets: one (batch, head)'s rows up to S + 128 (the last
    key block's padding) within 2^31 bytes of bf16, and at most 2^31 - 1 (batch, head)
    pairs (the same limits ``rk_attention_forward`` checks before launching)."""
    b, h, s, d = shape
    return ((s + 128) * stride[2] + d) * 2 < 2**31 and b * h <= 0x7FFFFFFF


def attention_supported(q: Tensor, k: Tensor, v: Tensor) -> bool:
    if not (q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 4):
        return False
    if k.shape != q.shape or v.shape != q.shape or k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    if q.shape[-1] not in (64, 128):
        return False
    for t in (q, k, v):
        if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:3]):
            return False
        if not _extent_fits(tuple(t.shape), t.stride()):
            return False
    return True


class CausalAttentionFn(torch.autograd.Function):
    """o = causal softmax(q k^T / sqrt(D)) v: HIP forward, torch's memory-efficient backward."""

    @staticmethod
    def forward(ctx, q: Tensor, k: Tensor, v: Tensor) -> Tensor:
        scale = 1.0 / math.sqrt(q.shape[-1])
        out, lse = ratchet().attention_forward(q, k, v, scale)
        ctx.save_for_backward(q, k, v, out, lse)
        return out

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        q, k, v, out, lse = ctx.saved_tensors
        seed, offset = _philox_placeholders()
        dq, dk, dv, _ = torch.ops.aten._scaled_dot_product_efficient_attention_backward(
            grad_out, q, k, v, None, out, lse, seed, offset, 0.0,
            [True, True, True, False], True)
        return dq, dk, dv


def causal_attention(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """``F.scaled_dot_product_attention(q, k, v, is_causal=True)``: the HIP forward where it
    applies, torch's otherwise."""
    if attention_supported(q, k, v):
        return CausalAttentionFn.apply(q, k, v)
    return F.scaled_dot_product_attention(q, k, v, is_causal=True)
