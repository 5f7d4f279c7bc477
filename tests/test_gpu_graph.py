"""HIP-graph replay of the int8 ratchet-linear training step.

The whole step (per-token quant, int8 forward, SR-quantized int8 grad_input, BF16
grad_weight, fused update) is captured once and replayed. Every replay must equal an
eager step of an identical layer on the same inputs: forward output, grad_input, packed
state and move counts, bit for bit, with eager work and synchronizations between the
replays.
"""

from __future__ import annotations

import pytest
import torch

from local_ai_training import ratchet as ratchet_mod
from local_ai_training.int8_matmul import quantize_rows_into
from local_ai_training.ratchet import DiscreteRatchetLinear

pytestmark = pytest.mark.gpu


def _layer(k: int, n: int, device) -> DiscreteRatchetLinear:
    torch.manual_seed(7)
    return DiscreteRatchetLinear(k, n, max_code=2, matmul_mode="int8", int8_backward=True,
                                 fuse_backward_update=True).to(device).train()


def test_graph_replays_match_eager_steps(cuda, monkeypatch):
    # The SR seed is drawn on the host once per backward; inside a graph it is the value
    # drawn at capture time, so both paths use one fixed seed here.
    monkeypatch.setattr(ratchet_mod, "_sr_seed", lambda: 424242)
    m, k, n = 1024, 512, 768
    eager, graphed = _layer(k, n, cuda), _layer(k, n, cuda)
    assert torch.equal(eager.packed, graphed.packed)
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(cuda)
    g = (torch.randn(m, n, generator=gen) * 1e-2).to(torch.bfloat16).to(cuda)

    def make_inputs():
        xi = x.clone().requires_grad_(True)
        return xi, torch.empty(m, k, dtype=torch.int8, device=cuda), \
            torch.empty(m, dtype=torch.float32, device=cuda)

    xe, qe, se = make_inputs()
    xg, qg, sg = make_inputs()
    held = {}

    def step(layer, xi, qi, si):
        xi.grad = None
        quantize_rows_into(xi.detach(), qi, si)
        out = layer(xi, inputs_int8=qi, inputs_scale=si)
        out.backward(g)
        stats = layer.ratchet_update(validate=False)
        return out, stats

    side = torch.cuda.Stream(device=cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        for _ in range(2):
            step(graphed, xg, qg, sg)
    torch.cuda.current_stream(cuda).wait_stream(side)
    for _ in range(2):
        step(eager, xe, qe, se)
    torch.cuda.synchronize()
    assert torch.equal(eager.packed, graphed.packed)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        held["out"], held["stats"] = step(graphed, xg, qg, sg)
    for replay in range(3):
        graph.replay()
        out_e, stats_e = step(eager, xe, qe, se)
        torch.cuda.synchronize()
        assert torch.equal(held["out"].view(torch.int16), out_e.view(torch.int16)), replay
        assert torch.equal(xg.grad.view(torch.int16), xe.grad.view(torch.int16)), replay
        assert torch.equal(graphed.packed, eager.packed), replay
        got = [int(held["stats"].positive_moves), int(held["stats"].negative_moves)]
        want = [int(stats_e.positive_moves), int(stats_e.negative_moves)]
        assert got == want, replay
