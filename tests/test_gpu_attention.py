"""The HIP causal-attention forward (``rk_attention_forward``, ``attention.py``) against the
forward it replaces, ``F.scaled_dot_product_attention(q, k, v, is_causal=True)``
(reference ``model.py:117-123``).

Checked against the float64 softmax on the CPU (the mathematical values: o within one bf16
rounding of the output plus the bf16 rounding of the probabilities, lse within float32
rounding), against torch's own memory-efficient forward on the GPU, and through the backward
(torch's memory-efficient backward fed our o and lse) against torch's whole attention.
Shapes: the 25M (B 32, H 8, S 512, D 64) and 1B (B 8, H 16, S 1024, D 128) attention with the
model's strided q/k/v views, and ragged sequence lengths.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from local_ai_training.attention import CausalAttentionFn, attention_supported
from local_ai_training.ops import ratchet

pytestmark = pytest.mark.gpu


def qkv_views(b, h, s, d, cuda, seed, scale=1.0):
    """q, k, v as the model makes them: chunks of one [B, S, 3C] tensor, viewed as heads."""
    g = torch.Generator().manual_seed(seed)
    c = h * d
    qkv = (torch.randn(b, s, 3 * c, generator=g) * scale).to(torch.bfloat16).to(cuda)
    q, k, v = qkv.chunk(3, dim=-1)
    return tuple(t.view(b, s, h, d).transpose(1, 2) for t in (q, k, v))


def reference(q, k, v):
    """float64 causal attention and log-sum-exp on the CPU."""
    qd, kd, vd = (t.detach().double().cpu() for t in (q, k, v))
    s = qd.shape[2]
    scores = (qd @ kd.transpose(-1, -2)) / math.sqrt(qd.shape[-1])
    mask = torch.ones(s, s, dtype=torch.bool).tril()
    scores = scores.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    return torch.softmax(scores, dim=-1) @ vd, lse


def check_forward(q, k, v):
    o, lse = ratchet().attention_forward(q, k, v, 1.0 / math.sqrt(q.shape[-1]))
    ref_o, ref_lse = reference(q, k, v)
    assert o.shape == q.shape and o.dtype == torch.bfloat16 and lse.shape == q.shape[:3]
    got = o.double().cpu()
    vmax = v.detach().double().abs().amax(dim=2, keepdim=True).cpu()  # [B, H, 1, D]
    # bf16 output rounding (2^-9 relative) + bf16 probabilities (2^-9 of sum p |v| <= max |v|)
    err = (got - ref_o).abs()
    assert bool((err <= 2.0 ** -8 * ref_o.abs() + 2.0 ** -8 * vmax + 1e-6).all()), \
        float((err / vmax.clamp_min(1e-9)).max())
    lerr = (lse.double().cpu() - ref_lse).abs()
    assert float(lerr.max()) <= 2e-5 * max(1.0, float(ref_lse.abs().max()))
    return o, lse


@pytest.mark.parametrize("b,h,s,d", [(32, 8, 512, 64), (8, 16, 1024, 128)])
def test_training_shapes_against_float64(cuda, b, h, s, d):
    print(f"attention forward {b}x{h}x{s}x{d}", flush=True)
    q, k, v = qkv_views(b, h, s, d, cuda, seed=s + d)
    assert attention_supported(q, k, v)
    check_forward(q, k, v)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("s", [1, 7, 64, 100, 129, 300])
def test_ragged_lengths_against_float64(cuda, s, d):
    print(f"attention forward ragged S={s} D={d}", flush=True)
    q, k, v = qkv_views(2, 3, s, d, cuda, seed=s * d, scale=2.0)
    check_forward(q, k, v)


def test_contiguous_inputs_and_large_scores(cuda):
    g = torch.Generator().manual_seed(5)
    q, k, v = ((torch.randn(2, 2, 200, 64, generator=g) * 6).to(torch.bfloat16).to(cuda)
               for _ in range(3))
    check_forward(q, k, v)


def test_matches_torch_forward_and_output_layout(cuda):
    q, k, v = qkv_views(4, 8, 512, 64, cuda, seed=9)
    o, lse = ratchet().attention_forward(q, k, v, 1.0 / 8.0)
    ref = torch.ops.aten._scaled_dot_product_efficient_attention(q, k, v, None, True, 0.0, True)
    assert o.stride() == ref[0].stride()  # [B, S, H, D] memory, as torch's forward writes
    diff = (o.float() - ref[0].float()).abs()
    assert float(diff.max()) <= 2.0 ** -6 * float(ref[0].float().abs().max())
    assert float((lse - ref[1]).abs().max()) <= 1e-4


@pytest.mark.parametrize("b,h,s,d", [(4, 8, 512, 64), (2, 16, 1024, 128), (2, 3, 129, 64)])
def test_gradients_match_torch_attention(cuda, b, h, s, d):
    """The HIP forward with torch's memory-efficient backward against torch's attention
    (the efficient kernel's forward and backward), same inputs and output gradient."""
    print(f"attention backward {b}x{h}x{s}x{d}", flush=True)
    q, k, v = qkv_views(b, h, s, d, cuda, seed=3 * s)
    go = torch.randn(b, h, s, d, generator=torch.Generator().manual_seed(4)).to(
        torch.bfloat16).to(cuda)
    grads = []
    for ours in (True, False):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        if ours:
            out = CausalAttentionFn.apply(qq, kk, vv)
        else:
            with torch.nn.attention.sdpa_kernel([torch.nn.attention.SDPBackend.EFFICIENT_ATTENTION]):
                out = F.scaled_dot_product_attention(qq, kk, vv, is_causal=True)
        out.backward(go)
        grads.append((out.detach().float(), qq.grad.float(), kk.grad.float(), vv.grad.float()))
    for mine, theirs in zip(*grads):
        scale = float(theirs.abs().max())
        assert float((mine - theirs).abs().max()) <= 2e-2 * scale


def test_runs_repeat_bit_for_bit(cuda):
    q, k, v = qkv_views(4, 8, 512, 64, cuda, seed=11)
    a = ratchet().attention_forward(q, k, v, 0.125)
    b = ratchet().attention_forward(q, k, v, 0.125)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_unsupported_inputs_fall_back(cuda):
    from local_ai_training.attention import causal_attention

    q = torch.randn(1, 2, 16, 32, device=cuda, dtype=torch.bfloat16)  # D = 32
    assert not attention_supported(q, q, q)
    out = causal_attention(q, q, q)
    assert torch.equal(out, F.scaled_dot_product_attention(q, q, q, is_causal=True))


def test_model_training_with_the_hip_forward(cuda):
    """A small int8 model: the HIP forward against torch's in the model's attention, the same
    forward loss within rounding, and three training steps that track each other."""
    import local_ai_training.model as model_mod
    from local_ai_training.model import ModelConfig, build_seeded_model
    from local_ai_training.training import training_step

    cfg = ModelConfig(vocab_size=256, block_size=128, n_layer=2, n_head=4, n_embd=256,
                      matmul_mode="int8", int8_backward=True)
    g = torch.Generator().manual_seed(7)
    tokens = torch.randint(0, 256, (8, 129), generator=g).to(cuda)
    runs = {}
    try:
        for hip in (True, False):
            model_mod.hip_attention_forward = hip
            model = build_seeded_model(cfg, max_code=2, seed=3).to(cuda).train()
            opt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=0.0)
            torch.manual_seed(2)
            losses = [float(training_step(model, opt, tokens[:, :-1], tokens[:, 1:])[0])
                      for _ in range(3)]
            runs[hip] = losses
    finally:
        model_mod.hip_attention_forward = True
    assert math.isclose(runs[True][0], runs[False][0], rel_tol=1e-3)
    assert all(math.isclose(a, b, rel_tol=2e-2) for a, b in zip(runs[True], runs[False]))
