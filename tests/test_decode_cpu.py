"""KV-cache logic of the decode path on the CPU (fp32 model, torch arithmetic only):
prefill + one-token steps reproduce the full-window forward at every position (the
reference's computation, generate.py:183-201), the cache refuses to outgrow block_size,
and generate() validates its arguments like the reference."""

from __future__ import annotations

import pytest
import torch

from local_ai_training.generate import generate
from local_ai_training.model import ModelConfig, build_seeded_model


def _model():
    config = ModelConfig(vocab_size=64, block_size=32, n_layer=2, n_head=4, n_embd=64,
                         matmul_mode="fp32")
    return build_seeded_model(config, max_code=2, seed=3).eval()


def test_cached_decode_reproduces_the_full_window_forward():
    model = _model()
    tokens = torch.randint(0, 64, (2, 30), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        full, _ = model(tokens)
    cache = model.new_cache(2)
    logits = model.prefill(tokens[:, :5], cache)
    torch.testing.assert_close(logits, full[:, 4], rtol=1e-5, atol=1e-5)
    for t in range(5, 30):
        logits = model.decode_step(tokens[:, t:t + 1], cache)
        torch.testing.assert_close(logits, full[:, t], rtol=1e-5, atol=1e-5)
    assert cache.length == 30 and int(cache.pos) == 30
    # a prompt appended in two chunks (explicit causal mask against the cache)
    cache2 = model.new_cache(2)
    model.prefill(tokens[:, :12], cache2)
    torch.testing.assert_close(model.prefill(tokens[:, 12:20], cache2), full[:, 19],
                               rtol=1e-5, atol=1e-5)


def test_bfloat16_cache_stores_bfloat16_and_returns_the_activation_dtype():
    model = _model()
    tokens = torch.randint(0, 64, (2, 20), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        full, _ = model(tokens)
    cache = model.new_cache(2, dtype=torch.bfloat16)
    logits = model.prefill(tokens[:, :6], cache)
    assert cache.keys[0].dtype == torch.bfloat16 and logits.dtype == torch.float32
    for t in range(6, 20):
        logits = model.decode_step(tokens[:, t:t + 1], cache)
        scale = float(full[:, t].abs().max())
        assert float((logits - full[:, t]).abs().max()) <= 3e-2 * scale, t
    # the stored keys are the bfloat16 rounding of the float32 keys
    ref = model.new_cache(2)
    model.prefill(tokens, ref)
    torch.testing.assert_close(cache.keys[1][:, :, :20].float(),
                               ref.keys[1][:, :, :20].to(torch.bfloat16).float(),
                               rtol=1e-2, atol=1e-2)


def test_cache_bounds():
    model = _model()
    with pytest.raises(ValueError, match="outgrow block_size"):
        model.new_cache(1, max_len=33)
    cache = model.new_cache(1, max_len=8)
    model.prefill(torch.zeros((1, 8), dtype=torch.long), cache)
    with pytest.raises(ValueError, match="KV cache is full"):
        model.prefill(torch.zeros((1, 1), dtype=torch.long), cache)


def test_generate_greedy_matches_window_recompute_and_validates():
    model = _model()
    vocabulary = tuple(chr(48 + i) for i in range(64))
    prompt = "".join(vocabulary[i] for i in (1, 5, 9, 2))
    out = generate(model, vocabulary, prompt, max_new_tokens=40, temperature=0.0)
    assert len(out) == 40
    # the reference's loop: full (cropped) window forward per token
    ids = [vocabulary.index(c) for c in prompt]
    for expected in out:
        window = torch.tensor([ids[-32:]])
        with torch.no_grad():
            logits, _ = model(window)
        nxt = int(logits[0, -1].argmax())
        assert vocabulary[nxt] == expected
        ids.append(nxt)
    with pytest.raises(ValueError, match="non-negative"):
        generate(model, vocabulary, prompt, max_new_tokens=1, temperature=-1.0)
    assert generate(model, vocabulary, "", max_new_tokens=3, temperature=0.0) != ""
