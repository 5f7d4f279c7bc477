"""The training loss as HIP kernels: ``F.cross_entropy(logits, targets)`` (mean reduction,
``ignore_index``), the loss line of the reference model (``model.py:249``), which the
training loop runs under bf16 autocast (``train.py:258-259``).

torch computes it as log_softmax (a [M, V] float32 result) then nll_loss, and its backward
fills a [M, V] gradient with zeros, scatters the nll gradient into it, and runs the
log_softmax backward over both. Here the forward reads the logits once and keeps three
floats per row (max, log of the sum of exponentials, the row's loss); the backward reads
the logits once more and writes the gradient once, in the logits' dtype. For bfloat16
logits (the int8 lm_head's output, whose float32 form is a widened bfloat16 value) the
gradient is bfloat16: the lm_head's backward reads it as bfloat16 anyway
(``ratchet.py:136-162``: ``grad_output.to(bfloat16)`` for grad_input and grad_weight).

The arithmetic is torch's, restated per row: out_j = (x_j - max) - log(sum exp(x_j - max)),
loss = mean over counted rows of -out_t; grad_j = [j == t] g - exp(out_j) * g with
g = -(grad_loss / count). Sums run in a fixed order, so results repeat from run to run; they
differ from torch's by float reassociation only. ``ignore_index`` rows count for nothing and
get zero gradient; a target outside [0, V) other than ``ignore_index`` gives a NaN loss.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from .ops import ratchet


def cross_entropy_supported(logits: Tensor, targets: Tensor) -> bool:
    """Whether the HIP kernels take these operands: GPU float32 / bfloat16 logits [M, V]
    with unit column stride, V and the row stride multiples of one 16-byte vector, 16-byte
    aligned, and int64 targets [M]."""
    if not (logits.is_cuda and logits.dim() == 2 and targets.dim() == 1):
        return False
    if logits.dtype not in (torch.float32, torch.bfloat16) or targets.dtype != torch.int64:
        return False
    m, v = logits.shape
    per_vec = 16 // logits.element_size()
    ld = logits.stride(0) if m > 1 else v
    return (targets.shape[0] == m and v > 0 and logits.stride(1) == 1 and v % per_vec == 0
            and ld % per_vec == 0 and logits.data_ptr() % 16 == 0
            and targets.device == logits.device)


class CrossEntropyFn(torch.autograd.Function):
    """Mean token cross-entropy over logits [M, V]; the gradient has the logits' dtype."""

    @staticmethod
    def forward(ctx, logits: Tensor, targets: Tensor, ignore_index: int) -> Tensor:
        loss, stats, count = ratchet().cross_entropy_forward(logits, targets, ignore_index)
        ctx.save_for_backward(logits, targets, stats, count)
        ctx.ignore_index = ignore_index
        return loss

    @staticmethod
    def backward(ctx, grad_loss: Tensor):
        logits, targets, stats, count = ctx.saved_tensors
        grad = ratchet().cross_entropy_backward(grad_loss, logits, targets, stats, count,
                                                ctx.ignore_index)
        return grad, None, None


def cross_entropy(logits: Tensor, targets: Tensor, ignore_index: int = -100) -> Tensor:
    """``F.cross_entropy(logits, targets, ignore_index=ignore_index)`` (mean reduction) for
    logits [M, V] and int64 class targets [M]: the HIP kernels where they apply, torch's own
    loss otherwise (CPU tensors, unaligned shapes)."""
    if cross_entropy_supported(logits, targets):
        return CrossEntropyFn.apply(logits, targets, ignore_index)
    return F.cross_entropy(logits, targets, ignore_index=ignore_index)
