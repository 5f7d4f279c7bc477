"""HIP-graph replay of the int8 ratchet-linear training step.

The whole step (per-token quant, int8 forward, SR-quantized int8 grad_input, BF16
grad_weight, fused update) is captured once and replayed. The SR seed of each replay is
read from a device slot that the host fills before the replay with the draw an eager step
would make (CapturedSeeds), so replays take fresh random bits. Every replay must equal an
eager step of an identical layer on the same inputs with the same host RNG state: forward
output, grad_input, packed state and move counts, bit for bit, with eager work and
synchronizations between the replays.
"""

from __future__ import annotations

import pytest
import torch

from local_ai_training.int8_matmul import CapturedSeeds, quantize_rows, quantize_rows_colscaled
from local_ai_training.ratchet import DiscreteRatchetLinear

pytestmark = pytest.mark.gpu


def _layer(k: int, n: int, device) -> DiscreteRatchetLinear:
    torch.manual_seed(7)
    return DiscreteRatchetLinear(k, n, max_code=2, matmul_mode="int8", int8_backward=True,
                                 fuse_backward_update=True).to(device).train()


def _setup(cuda, m=1024, k=512, n=768):
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(cuda)
    g = (torch.randn(m, n, generator=gen) * 1e-2).to(torch.bfloat16).to(cuda)

    def step(layer, xi):
        xi.grad = None
        qi, si = quantize_rows(xi.detach())
        out = layer(xi, inputs_int8=qi, inputs_scale=si)
        out.backward(g)
        return out, layer.ratchet_update(validate=False)

    return x, step


def _capture(layer, xg, step, seeds, device):
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for _ in range(2):
            step(layer, xg)
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with seeds.recording(), torch.cuda.graph(graph):
        held = step(layer, xg)
    return graph, held


def test_graph_replays_match_eager_steps_with_fresh_seeds(cuda):
    m, k, n = 1024, 512, 768
    x, step = _setup(cuda, m, k, n)
    eager, graphed = _layer(k, n, cuda), _layer(k, n, cuda)
    xe, xg = x.clone().requires_grad_(True), x.clone().requires_grad_(True)
    torch.manual_seed(11)
    seeds = CapturedSeeds(cuda)
    graph, (out_g, stats_g) = _capture(graphed, xg, step, seeds, cuda)
    torch.manual_seed(11)
    for _ in range(2):
        step(eager, xe)
    torch.cuda.synchronize()
    assert torch.equal(eager.packed, graphed.packed)
    assert seeds.used == 1  # one stochastic rounding per step: the layer's grad_input

    drawn = []
    for replay in range(3):
        torch.manual_seed(100 + replay)
        drawn += seeds.refill()
        graph.replay()
        torch.manual_seed(100 + replay)
        out_e, stats_e = step(eager, xe)
        torch.cuda.synchronize()
        assert eager.last_sr_seed == drawn[-1], replay
        assert torch.equal(out_g.view(torch.int16), out_e.view(torch.int16)), replay
        assert torch.equal(xg.grad.view(torch.int16), xe.grad.view(torch.int16)), replay
        assert torch.equal(graphed.packed, eager.packed), replay
        got = [int(stats_g.positive_moves), int(stats_g.negative_moves)]
        want = [int(stats_e.positive_moves), int(stats_e.negative_moves)]
        assert got == want, replay
    assert len(set(drawn)) == 3


def test_replays_with_different_seeds_round_differently(cuda):
    # Same state, same inputs, two replays: the SR bits follow the slot's seed (equal seeds
    # give equal grad_input, different seeds a different one).
    m, k, n = 512, 256, 384
    x, step = _setup(cuda, m, k, n)
    layer = _layer(k, n, cuda)
    xg = x.clone().requires_grad_(True)
    seeds = CapturedSeeds(cuda)
    graph, _ = _capture(layer, xg, step, seeds, cuda)
    start = layer.packed.clone()

    def replay_with(seed_state: int) -> torch.Tensor:
        layer.packed.copy_(start)
        torch.manual_seed(seed_state)
        seeds.refill()
        graph.replay()
        torch.cuda.synchronize()
        return xg.grad.clone()

    a, b, c = replay_with(1), replay_with(2), replay_with(1)
    assert torch.equal(a.view(torch.int16), c.view(torch.int16))
    assert not torch.equal(a, b)


@pytest.mark.parametrize("fused_adamw", [False, True])
def test_captured_training_step_equals_eager_steps(cuda, fused_adamw):
    # The model's whole training step (autocast forward, backward with the fused updates,
    # ratchet_update, capturable AdamW: torch's foreach form, or its fused kernel as the
    # benchmark uses) replayed as a graph: losses, every ratchet state and every float
    # parameter equal an eager run of the same steps with the same host RNG.
    from local_ai_training.model import ModelConfig, build_seeded_model
    from local_ai_training.training import CapturedTrainingStep, training_step

    config = ModelConfig(vocab_size=256, block_size=64, n_layer=2, n_head=4, n_embd=128,
                         matmul_mode="int8", int8_backward=True)
    gen = torch.Generator().manual_seed(4)
    batches = [torch.randint(0, 256, (8, 65), generator=gen).to(cuda) for _ in range(6)]
    runs = []
    for graphed in (False, True):
        model = build_seeded_model(config, max_code=2, seed=21).to(cuda).train()
        optimizer = torch.optim.AdamW(model.parameters(), lr=3e-3, weight_decay=0.0,
                                      capturable=True, fused=fused_adamw)
        torch.manual_seed(8)
        losses = []
        if graphed:
            step = CapturedTrainingStep(model, optimizer, batches[0][:, :-1],
                                        batches[0][:, 1:], warmup_steps=2)
            losses += [None, None]  # the two warm-up steps ran batch 0 eagerly
            for batch in batches[2:]:
                losses.append(float(step(batch[:, :-1], batch[:, 1:])))
        else:
            for index, batch in enumerate(batches):
                data = batches[0] if index < 2 else batch
                loss, _ = training_step(model, optimizer, data[:, :-1], data[:, 1:],
                                        autocast_cache=False)
                losses.append(float(loss))
            losses[:2] = [None, None]
        torch.cuda.synchronize()
        states = [m.packed.clone() for m in model.modules() if isinstance(m, DiscreteRatchetLinear)]
        runs.append((losses, states, [p.detach().clone() for p in model.parameters()]))
    (le, se, pe), (lg, sg, pg) = runs
    assert le == lg
    assert all(torch.equal(a, b) for a, b in zip(se, sg))
    assert all(torch.equal(a, b) for a, b in zip(pe, pg))


def test_stochastic_rounding_in_a_capture_needs_a_seed_source(cuda):
    # A host seed drawn at capture time would be replayed forever: the call raises before
    # it launches anything (the capture then ends empty).
    g = torch.randn(64, 128, device=cuda)
    col = torch.ones(128, device=cuda)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="seed source"):
        with torch.cuda.graph(graph):
            quantize_rows_colscaled(g, col, stochastic=True)
    torch.cuda.synchronize()
