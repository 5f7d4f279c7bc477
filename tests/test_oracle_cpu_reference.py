"""The CPU baselines' restatement of the reference's fp32 training path (oracle/cpu_reference.py):
its fused-backward update is the oracle's integer update on the same normalized gradient, and the
tiny-model step trains (finite, falling loss; codes move)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import update as oupd
from oracle.cpu_reference import TinyRatchetGPT, _RatchetLinearFn, fp32_ratchet_linear_step


def test_fused_backward_update_equals_the_oracle_update():
    gen = torch.Generator().manual_seed(3)
    n, k, m, mc = 300, 48, 40, 2
    code = torch.randint(-mc, mc + 1, (n, k), generator=gen)
    packed = (((code + mc) & 0x0F) | (7 << 4)).to(torch.uint8)
    start = packed.clone()
    scale = torch.rand(n, generator=gen) * 0.08 + 0.02
    x = torch.randn(m, k, generator=gen, requires_grad=True)
    g = torch.randn(m, n, generator=gen)
    out = _RatchetLinearFn.apply(x, packed, scale, mc)
    out.backward(g)
    # the same 256-row tiles and the same float32 normalization, then the oracle's integer
    # update (pinned by the reference's golden vectors): the states must agree exactly
    gw = g.t() @ x.detach()
    want = start.numpy().copy()
    for t0 in range(0, n, 256):
        t1 = min(t0 + 256, n)
        tile = gw[t0:t1]
        z = tile / (tile.square().mean(dim=1, keepdim=True).sqrt() + 1e-8)
        want[t0:t1], _ = oupd.update_core(want[t0:t1], z.numpy(), mc, 8)
    assert int((want != start.numpy()).sum()) > 0
    assert np.array_equal(packed.numpy(), want)
    ref_gi = g @ (((start.to(torch.int16) & 0x0F) - mc).float() * scale[:, None])
    assert torch.allclose(x.grad, ref_gi, atol=1e-5)


def test_op_step_and_tiny_model_train():
    gen = torch.Generator().manual_seed(4)
    packed = (((torch.randint(-2, 3, (64, 32), generator=gen) + 2) & 0x0F) | (7 << 4)).to(torch.uint8)
    before = packed.clone()
    out, gi, moves = fp32_ratchet_linear_step(torch.randn(128, 32, generator=gen), packed,
                                              torch.rand(64, generator=gen) * 0.08 + 0.02,
                                              torch.randn(128, 64, generator=gen), 2, threshold=1)
    assert out.shape == (128, 64) and gi.shape == (128, 32)
    assert int(moves) == int(((before & 0x0F) != (packed & 0x0F)).sum())

    model = TinyRatchetGPT(256, 32, 4, 1, 64, 16, 2, seed=5)
    packs = [m.packed.clone() for m in model.modules() if hasattr(m, "packed")]
    opt = torch.optim.AdamW([p for p in model.parameters() if p.requires_grad], lr=1e-2)
    tokens = torch.randint(0, 256, (4, 17), generator=gen)
    losses = []
    for _ in range(6):
        opt.zero_grad(set_to_none=True)
        loss = model(tokens[:, :-1], tokens[:, 1:])
        loss.backward()
        opt.step()
        losses.append(float(loss.detach()))
    assert all(np.isfinite(losses)) and losses[-1] < losses[0]
    after = [m.packed for m in model.modules() if hasattr(m, "packed")]
    assert any(not torch.equal(a, b) for a, b in zip(packs, after))
