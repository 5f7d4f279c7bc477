"""One training step of the ratchet transformer, run eagerly or replayed as a HIP graph.

``training_step`` is the body of the reference's training loop (``train.py:255-275``):
zero the float gradients, bf16-autocast forward and loss, stop on a non-finite loss,
backward (every ratchet layer updates its packed state inside it), ``ratchet_update``
for the statistics, then the optimizer step on the float parameters.

``CapturedTrainingStep`` captures that step once into a HIP graph and replays it. Every
replay launches the same kernels on the same buffers, so the Python autograd and launch
overhead of the eager step is gone; the batch is copied into fixed input buffers first.
What a replay keeps identical to an eager step:

* the stochastic-rounding seeds: each int8-backward layer reads its seed from a device slot
  that is filled before the replay with the draws an eager step would make from the CPU
  generator, in the same order (``int8_matmul.CapturedSeeds``), so the host RNG stream and
  the random bits match an eager run;
* the optimizer: it must be built with ``capturable=True`` (its step count lives on the
  device), the form torch requires for graph capture;
* the numerics: autocast runs with its cast cache off (``cache_enabled=False``), which
  changes no value.

A model whose token-embedding gradient would come from torch's sort-based backward is
refused before anything runs (``RatchetGPT.embedding_backward_is_sort_based``): that
backward records a memset node in the graph, and such nodes are not safe on replays.

The warm-up steps that precede the capture are real training steps.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .int8_matmul import CapturedSeeds
from .model import RatchetGPT
from .ratchet import RatchetUpdateStats


def training_step(model: RatchetGPT, optimizer: torch.optim.Optimizer, inputs: Tensor,
                  targets: Tensor, *, validate: bool = False, check_finite: bool = True,
                  autocast_cache: bool = True) -> tuple[Tensor, RatchetUpdateStats]:
    """One step of the reference loop; returns (loss, update statistics). ``validate``
    checks the ratchet state and materializes the statistics (host syncs, the reference's
    eval cadence); ``check_finite`` raises FloatingPointError on a non-finite loss (one host
    sync, as the reference does every step)."""
    optimizer.zero_grad(set_to_none=True)
    with torch.autocast(device_type=inputs.device.type, dtype=torch.bfloat16,
                        cache_enabled=autocast_cache):
        _, loss = model(inputs, targets)
    if check_finite and not torch.isfinite(loss):
        model.discard_pending_gradients()
        raise FloatingPointError("non-finite training loss")
    loss.backward()
    stats = model.ratchet_update(validate=validate)
    optimizer.step()
    return loss, stats


class CapturedTrainingStep:
    """``training_step`` captured once as a HIP graph and replayed (see the module notes).

    ``inputs`` / ``targets`` give the batch shape (and are the first batch of the warm-up
    steps); each call copies its batch into the graph's input buffers, refills the SR seed
    slots and replays. The returned loss and ``stats`` are overwritten by the next call.
    """

    def __init__(self, model: RatchetGPT, optimizer: torch.optim.Optimizer, inputs: Tensor,
                 targets: Tensor, *, warmup_steps: int = 2) -> None:
        if model.embedding_backward_is_sort_based():
            # checked before any step runs: the capture would record that backward's memset
            # node (see RatchetGPT.embedding_backward_is_sort_based)
            raise RuntimeError(
                "CapturedTrainingStep refuses this model: its token-embedding gradient would "
                "come from torch's sort-based embedding backward, whose memset node is not "
                "safe in a replayed graph; use an nn.Embedding with hip_embedding_backward "
                "(no padding_idx, max_norm, sparse or scale_grad_by_freq; width a multiple "
                "of 4, at most 4096) or run the step eagerly")
        if not inputs.is_cuda:
            raise RuntimeError("CapturedTrainingStep requires CUDA (a ROCm GPU)")
        if not all(group.get("capturable", False) for group in optimizer.param_groups):
            raise ValueError("graph capture needs an optimizer built with capturable=True")
        self.model, self.optimizer = model, optimizer
        self.inputs, self.targets = inputs.clone(), targets.clone()
        self.seeds = CapturedSeeds(inputs.device)
        device = inputs.device

        def step():
            return training_step(model, optimizer, self.inputs, self.targets,
                                 check_finite=False, autocast_cache=False)

        side = torch.cuda.Stream(device=device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            for _ in range(max(warmup_steps, 1)):
                step()
        torch.cuda.current_stream(device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with self.seeds.recording(), torch.cuda.graph(self.graph):
            self.loss, self.stats = step()

    def __call__(self, inputs: Tensor | None = None, targets: Tensor | None = None) -> Tensor:
        if inputs is not None:
            self.inputs.copy_(inputs)
        if targets is not None:
            self.targets.copy_(targets)
        self.seeds.refill()
        self.graph.replay()
        return self.loss
