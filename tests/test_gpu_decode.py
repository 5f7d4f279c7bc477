"""KV-cached decoding (RatchetGPT.prefill / decode_step, generate.DecodeGraph) against the
reference's way of producing a token: the full-window forward, read at the last position
(generate.py:183-201).

The int8 GEMMs are exact, but attention over a cache sums in a different order than the
full-window attention, so activations can differ in the last float bits and a quantized
activation can move by one step; logits are compared at rel 1e-2 of their scale and the
greedy token must agree on almost every position. Graph replays run the same kernels on
the same data as eager decode steps and must match them bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from local_ai_training.generate import DecodeGraph, generate
from local_ai_training.model import ModelConfig, build_seeded_model

pytestmark = pytest.mark.gpu


def _model(cuda, mode="int8", **kw):
    config = ModelConfig(vocab_size=256, block_size=64, n_layer=2, n_head=4, n_embd=128,
                         matmul_mode=mode, **kw)
    return build_seeded_model(config, max_code=2, seed=11).to(cuda).eval()


def _close(got, want, rel=1e-2):
    scale = float(want.abs().max())
    return float((got - want).abs().max()) <= rel * scale


@pytest.mark.parametrize("mode", ["int8", "fp32"])
def test_prefill_and_decode_match_the_full_window_forward(cuda, mode):
    model = _model(cuda, mode)
    gen = torch.Generator().manual_seed(5)
    tokens = torch.randint(0, 256, (3, 40), generator=gen).to(cuda)
    with torch.no_grad():
        full, _ = model(tokens)
    cache = model.new_cache(3)
    logits = model.prefill(tokens[:, :8], cache)
    assert cache.length == 8 and int(cache.pos.item()) == 8
    assert _close(logits, full[:, 7])
    agree = total = 0
    for t in range(8, 40):
        logits = model.decode_step(tokens[:, t:t + 1], cache)
        assert _close(logits, full[:, t]), t
        agree += int((logits.argmax(-1) == full[:, t].argmax(-1)).sum())
        total += 3
    assert agree >= 0.95 * total
    # a second prompt chunk at a nonzero start (explicit causal mask against the cache)
    cache2 = model.new_cache(3)
    model.prefill(tokens[:, :20], cache2)
    logits2 = model.prefill(tokens[:, 20:30], cache2)
    assert _close(logits2, full[:, 29])


def test_decode_graph_replays_equal_eager_steps(cuda):
    model = _model(cuda)
    gen = torch.Generator().manual_seed(6)
    tokens = torch.randint(0, 256, (2, 24), generator=gen).to(cuda)
    eager, graphed = model.new_cache(2), model.new_cache(2)
    model.prefill(tokens[:, :4], eager)
    model.prefill(tokens[:, :4], graphed)
    graph = DecodeGraph(model, graphed)
    for t in range(4, 24):
        want = model.decode_step(tokens[:, t:t + 1], eager)
        got = graph.step(tokens[:, t:t + 1])
        torch.cuda.synchronize()
        assert torch.equal(got, want), t
    assert graphed.length == eager.length == 24


def test_generate_is_graph_independent_and_crosses_the_window(cuda):
    model = _model(cuda)
    vocabulary = tuple(chr(0x100 + i) for i in range(256))
    prompt = "".join(vocabulary[i] for i in range(10))
    a = generate(model, vocabulary, prompt, max_new_tokens=70, temperature=0.0)
    b = generate(model, vocabulary, prompt, max_new_tokens=70, temperature=0.0, use_graph=True)
    assert len(a) == 70 and a == b
    c = generate(model, vocabulary, prompt, max_new_tokens=12, temperature=0.8, top_k=20,
                 seed=3)
    d = generate(model, vocabulary, prompt, max_new_tokens=12, temperature=0.8, top_k=20,
                 seed=3)
    assert len(c) == 12 and c == d
    with pytest.raises(ValueError, match="not in the model vocabulary"):
        generate(model, vocabulary, "?", max_new_tokens=1)
    with pytest.raises(ValueError, match="non-negative"):
        generate(model, vocabulary, prompt, max_new_tokens=-1)


def test_sliding_window_step_matches_the_reference_recompute(cuda):
    # A prompt longer than block_size: its last 64 tokens are prefilled (logits as the full
    # window forward's last position); the next token comes from the re-positioned window,
    # which is the reference's own computation, so it must be that forward's argmax.
    model = _model(cuda)
    vocabulary = tuple(chr(0x100 + i) for i in range(256))
    gen = torch.Generator().manual_seed(9)
    ids = torch.randint(0, 256, (80,), generator=gen).tolist()
    cache = model.new_cache(1)
    prefill = model.prefill(torch.tensor([ids[-64:]], device=cuda), cache)
    with torch.no_grad():
        full, _ = model(torch.tensor([ids[-64:]], device=cuda))
    assert _close(prefill, full[:, -1])
    prompt = "".join(vocabulary[i] for i in ids)
    out = generate(model, vocabulary, prompt, max_new_tokens=2, temperature=0.0)
    first = vocabulary.index(out[0])
    window = torch.tensor([(ids + [first])[-64:]], device=cuda)
    with torch.no_grad():
        logits, _ = model(window)
    assert out[1] == vocabulary[int(logits[0, -1].argmax())]
