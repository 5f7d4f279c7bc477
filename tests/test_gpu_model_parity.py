"""Model-level integer-state parity of the int8 ratchet transformer against the oracle.

The model trains as the reference's loop does (train.py:248-277): bf16 autocast forward,
backward with the ratchet update fused into it, AdamW on the float parameters, with
matmul_mode="int8" and int8_backward on. Every ratchet layer's step is recorded from the
real run (the GEMM and SR-quant calls of its autograd Function) and replayed by the oracle
with the float producers taken from the GPU (teacher forcing: the prologues' int8 rows and
scales, the upstream gradient, the bf16 weight gradient the update consumed):

  - forward GEMM output (bf16 bits; + the residual where the GEMM adds it),
  - SR-quantized gradient and its scales, for every int8-backward layer, with the seed the
    reference's order gives: one draw from the CPU generator per layer, in backward order
    (each block's contraction, expand, projection, qkv; the last block first), the lm_head
    excluded since it keeps the bf16 grad_input (int8_matmul.py:200, ratchet.py:125-141),
  - int8 grad_input,
  - the packed state after the update and the move counts.

Tiny config (2 layers, d 128, 4 heads, FFN 512, byte vocab 256, seq 64, batch 8; quinary
codes uniform, pressure 0, row scales U[0.02, 0.1]): every row, 100 steps. The 25M config:
sampled token rows and features of every layer, drawn afresh each step, 100 steps; the 1B
config likewise for 3 steps.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from local_ai_training import int8_matmul, ops
from local_ai_training import ratchet as ratchet_mod
from local_ai_training.model import ModelConfig, build_seeded_model
from local_ai_training.ratchet import DiscreteRatchetLinear, pack_code_pressure
from oracle import update as oupd
from parity import check_forward, check_grad_input, check_sr_quant, check_update, sample_rows

pytestmark = pytest.mark.gpu


class StepRecorder:
    """Records, per ratchet layer and step, the sampled rows of what its int8 GEMMs and SR
    quant consumed and produced (installed over the functions the autograd Function calls:
    the separate quant and GEMM, the quant of a gradient in parts, and the fused SR quant +
    grad_input, whose int8 codes are captured through its optional output)."""

    def __init__(self, model, token_rows: np.ndarray | None, seed: int) -> None:
        self.layers = {name: m for name, m in model.named_modules()
                       if isinstance(m, DiscreteRatchetLinear)}
        self.by_ptr = {m.packed.data_ptr(): name for name, m in self.layers.items()}
        self.token_rows = token_rows
        self.seed = seed
        self.reset()

    def reset(self):
        self.forward, self.sr, self.grad_input = {}, [], {}
        self._sr_by_q = {}

    def rows(self, m: int, device) -> torch.Tensor:
        rows = np.arange(m) if self.token_rows is None else self.token_rows
        return torch.from_numpy(rows).to(device)

    def install(self, monkeypatch):
        orig_mm = ratchet_mod.packed_int8_mm
        orig_res = ratchet_mod.packed_int8_mm_residual
        orig_t = ratchet_mod.packed_int8_mm_t
        orig_sr = ratchet_mod.quantize_rows_sr

        def mm(a, packed, max_code, a_scale, row_scale, out_dtype=torch.bfloat16):
            out = orig_mm(a, packed, max_code, a_scale, row_scale, out_dtype)
            r = self.rows(a.shape[0], a.device)
            self.forward[self.by_ptr[packed.data_ptr()]] = (a[r], a_scale[r], out[r], None)
            return out

        def mm_residual(a, packed, max_code, a_scale, row_scale, residual, out=None):
            r = self.rows(a.shape[0], a.device)
            res_rows = residual[r].clone()
            result = orig_res(a, packed, max_code, a_scale, row_scale, residual, out)
            self.forward[self.by_ptr[packed.data_ptr()]] = (a[r], a_scale[r], result[r],
                                                            res_rows)
            return result

        def sr(values, col_scale=None, *, bf16_out=None, row_offset=0, round_bf16=False):
            q, s, seed = orig_sr(values, col_scale, bf16_out=bf16_out, row_offset=row_offset,
                                 round_bf16=round_bf16)
            r = self.rows(values.shape[0], values.device)
            self._sr_by_q[q.data_ptr()] = len(self.sr)
            # the values as quantized: a float32 gradient taken as bf16 is the bf16 gradient
            # the reference's projection receives from its mixed-dtype residual add
            consumed = values[r].to(torch.bfloat16) if round_bf16 else values[r].clone()
            self.sr.append([None, consumed, seed, q[r], s[r]])
            return q, s, seed

        def mm_t(a, packed, max_code, a_scale, row_scale, out_dtype=torch.bfloat16):
            out = orig_t(a, packed, max_code, a_scale, row_scale, out_dtype)
            name = self.by_ptr[packed.data_ptr()]
            self.sr[self._sr_by_q[a.data_ptr()]][0] = name
            r = self.rows(a.shape[0], a.device)
            self.grad_input[name] = (a[r], a_scale[r], out[r])
            return out

        def sr_parts(parts, col_scale=None):
            q, s, seed = orig_sr_parts(parts, col_scale)
            r = self.rows(q.shape[0], q.device)
            self._sr_by_q[q.data_ptr()] = len(self.sr)
            self.sr.append([None, torch.cat(parts, dim=-1)[r], seed, q[r], s[r]])
            return q, s, seed

        orig_sr_parts = ratchet_mod.quantize_rows_sr_parts
        monkeypatch.setattr(ratchet_mod, "quantize_rows_sr_parts", sr_parts)
        monkeypatch.setattr(ratchet_mod, "packed_int8_mm", mm)
        monkeypatch.setattr(ratchet_mod, "packed_int8_mm_residual", mm_residual)
        monkeypatch.setattr(ratchet_mod, "packed_int8_mm_t", mm_t)
        monkeypatch.setattr(ratchet_mod, "quantize_rows_sr", sr)


def backward_order(model) -> list[str]:
    """The int8-backward layers in the order the reference's backward reaches them."""
    order = []
    for index in reversed(range(len(model.blocks))):
        prefix = f"blocks.{index}."
        order += [prefix + "feed_forward.contract", prefix + "feed_forward.expand",
                  prefix + "attention.projection", prefix + "attention.qkv"]
    return order


def make_model(cuda, *, vocab, block, n_layer, n_head, n_embd, ffn, max_code, seed,
               random_pressure=False):
    """The config's model with codes uniform in [-max_code, max_code], row scales
    U[0.02, 0.1] and pressure 0 (or uniform in [-7, 7], so that codes move from the first
    step on)."""
    config = ModelConfig(vocab_size=vocab, block_size=block, n_layer=n_layer, n_head=n_head,
                         n_embd=n_embd, ffn_hidden=ffn, matmul_mode="int8", int8_backward=True)
    model = build_seeded_model(config, max_code=max_code, seed=seed).to(cuda).train()
    gen = torch.Generator(device=cuda).manual_seed(seed + 1)
    for layer in model.modules():
        if isinstance(layer, DiscreteRatchetLinear):
            shape = tuple(layer.packed.shape)
            code = torch.randint(-max_code, max_code + 1, shape, generator=gen, device=cuda,
                                 dtype=torch.int8)
            pressure = (torch.randint(-7, 8, shape, generator=gen, device=cuda,
                                      dtype=torch.int8)
                        if random_pressure else torch.zeros_like(code))
            layer.packed.copy_(pack_code_pressure(code, pressure, max_code))
            layer._scale.copy_(torch.rand(layer.out_features, generator=gen, device=cuda)
                               * 0.08 + 0.02)
            layer.keep_weight_gradient = True
    return model


def run_parity(cuda, monkeypatch, model, tokens, steps, max_code, token_rows, feature_count):
    """Train `steps` steps, checking every layer against the oracle each step; returns the
    per-step losses. token_rows: the token rows checked (None: all); feature_count: how
    many output features (forward columns and update rows) and input features (grad_input
    columns) are checked per layer and step (None: all)."""
    recorder = StepRecorder(model, token_rows, seed=0)
    recorder.install(monkeypatch)
    optimizer = torch.optim.AdamW(model.parameters(), lr=3e-4, weight_decay=0.0)
    inputs, targets = tokens[:, :-1], tokens[:, 1:]
    order = backward_order(model)
    losses = []
    for step in range(steps):
        recorder.reset()
        # the checked rows (output features) and columns (input features) of each state,
        # copied before the step updates it in place
        picks, before = {}, {}
        for index, (name, layer) in enumerate(recorder.layers.items()):
            n, k = layer.packed.shape
            if feature_count is None:
                outs, ins = np.arange(n), np.arange(k)
            else:
                outs = sample_rows(n, feature_count, 31 * step + index)
                ins = sample_rows(k, feature_count, 57 * step + index)
            outs_t, ins_t = torch.from_numpy(outs).to(cuda), torch.from_numpy(ins).to(cuda)
            picks[name] = (outs, outs_t, ins_t)
            before[name] = (layer.packed[outs_t].cpu().numpy(),
                            layer.packed[:, ins_t].cpu().numpy())
        optimizer.zero_grad(set_to_none=True)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            _, loss = model(inputs, targets)
        rng = torch.get_rng_state()
        loss.backward()
        after_rng = torch.get_rng_state()
        stats = model.ratchet_update(validate=True)
        optimizer.step()
        losses.append(float(loss))

        # seeds: one CPU-generator draw per int8-backward layer, in backward order
        torch.set_rng_state(rng)
        want_seeds = [int(torch.randint(0, 2**31 - 1, (1,)).item()) for _ in order]
        assert torch.equal(torch.get_rng_state(), after_rng), f"step {step}: extra RNG draws"
        assert [entry[0] for entry in recorder.sr] == order, f"step {step}: SR order"
        assert [entry[2] for entry in recorder.sr] == want_seeds, f"step {step}: SR seeds"

        total = np.zeros(4, np.int64)
        for name, layer in recorder.layers.items():
            outs, outs_t, ins_t = picks[name]
            rows_before, cols_before = before[name]
            scale = layer.scale.detach().float().cpu().numpy()[outs]
            q, s, out, residual = recorder.forward[name]
            code_rows, _ = oupd.unpack(rows_before, max_code)
            check_forward(code_rows, scale, q, s, out[:, outs_t],
                          None if residual is None else residual[:, outs_t],
                          what=f"{name} step {step}")
            total += check_update(rows_before, layer.last_weight_gradient[outs_t],
                                  layer.packed[outs_t].cpu().numpy(), max_code,
                                  what=f"{name} step {step}")
        for name, g, seed, gq, gs in recorder.sr:
            layer = recorder.layers[name]
            _, _, ins_t = picks[name]
            scale = layer.scale.detach().float().cpu().numpy()
            rows = np.arange(inputs.numel()) if token_rows is None else token_rows
            check_sr_quant(g, scale, seed, rows, gq, gs, what=f"{name} step {step}")
            a, a_scale, gin = recorder.grad_input[name]
            code_cols, _ = oupd.unpack(before[name][1], max_code)
            check_grad_input(code_cols, a, a_scale, gin[:, ins_t], what=f"{name} step {step}")
        if feature_count is None:
            got = [stats.positive_moves, stats.negative_moves, stats.blocked_positive_moves,
                   stats.blocked_negative_moves]
            assert got == total.tolist(), f"step {step}: move counts"
        print(f"step {step}: loss {losses[-1]:.4f}, moves {int(stats.code_moves)} ok",
              flush=True)
    return losses


def test_tiny_config_hundred_steps_every_row_bit_exact(cuda, monkeypatch):
    model = make_model(cuda, vocab=256, block=64, n_layer=2, n_head=4, n_embd=128, ffn=512,
                       max_code=2, seed=1337)
    gen = torch.Generator().manual_seed(20)
    tokens = torch.randint(0, 256, (8, 65), generator=gen).to(cuda)
    torch.manual_seed(1234)
    losses = run_parity(cuda, monkeypatch, model, tokens, 100, 2, None, None)
    assert np.mean(losses[-10:]) < np.mean(losses[:10])


def zipf_tokens(batch, block, vocab, seed, device):
    rng = np.random.default_rng(seed)
    ids = (rng.zipf(1.1, size=batch * (block + 1)) - 1) % vocab
    return torch.from_numpy(ids.astype(np.uint16).astype(np.int64)).view(batch, block + 1).to(
        device)


# The 25M config for 100 steps (the reference's "bit-exact integer state after 100
# training steps" at a real training shape; every step checks freshly sampled rows and
# features of every layer), the 1B config for 3.
@pytest.mark.parametrize("config,steps", [("25M", 100), ("1B", 3)])
def test_training_config_sampled_rows_bit_exact(cuda, monkeypatch, config, steps):
    if config == "25M":
        shape = dict(vocab=8192, block=512, n_layer=8, n_head=8, n_embd=512, ffn=2048,
                     max_code=2)
        batch, token_rows, features = 32, 16, 64
    else:
        shape = dict(vocab=8192, block=1024, n_layer=24, n_head=16, n_embd=2048, ffn=5632,
                     max_code=3)
        batch, token_rows, features = 8, 8, 32
    print(f"{config} model, batch {batch}", flush=True)
    model = make_model(cuda, seed=1337, random_pressure=True, **shape)
    tokens = zipf_tokens(batch, shape["block"], shape["vocab"], 1337, cuda)
    rows = sample_rows(batch * shape["block"], token_rows, 7)
    torch.manual_seed(99)
    losses = run_parity(cuda, monkeypatch, model, tokens, steps, shape["max_code"], rows,
                        features)
    if steps >= 100:
        assert np.mean(losses[-10:]) < np.mean(losses[:10])
    del model
    torch.cuda.empty_cache()


def test_25m_training_steps_are_reproducible(cuda):
    # Two runs of the same seeded 25M training steps give identical losses and ratchet
    # states (every kernel of the step sums in a fixed order).
    shape = dict(vocab=8192, block=512, n_layer=8, n_head=8, n_embd=512, ffn=2048, max_code=2)
    tokens = zipf_tokens(32, 512, 8192, 1337, cuda)
    results = []
    for _ in range(2):
        model = make_model(cuda, seed=1337, random_pressure=True, **shape)
        optimizer = torch.optim.AdamW(model.parameters(), lr=3e-4, weight_decay=0.0)
        torch.manual_seed(5)
        losses = []
        for _ in range(4):
            optimizer.zero_grad(set_to_none=True)
            with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
                _, loss = model(tokens[:, :-1], tokens[:, 1:])
            loss.backward()
            model.ratchet_update(validate=False)
            optimizer.step()
            losses.append(float(loss))
        states = [layer.packed.clone() for layer in model.modules()
                  if isinstance(layer, DiscreteRatchetLinear)]
        results.append((losses, states, [p.detach().clone() for p in model.parameters()]))
        print(f"run losses {losses}", flush=True)
        del model, optimizer
    (l0, s0, p0), (l1, s1, p1) = results
    assert l0 == l1
    assert all(torch.equal(a, b) for a, b in zip(s0, s1))
    assert all(torch.equal(a, b) for a, b in zip(p0, p1))


def test_1b_training_steps_are_reproducible_in_deterministic_mode(cuda):
    # The 1B step (24 layers, d 2048, 16 heads, FFN 5632, seq 1024, batch 8, septenary
    # codes) run twice from the same seeds, two steps each: identical losses, ratchet states
    # and float parameters. Deterministic mode selects the flash attention backward (the
    # memory-efficient one's dq accumulation order varies at head size 128); every ratchet
    # kernel sums in a fixed order either way.
    shape = dict(vocab=8192, block=1024, n_layer=24, n_head=16, n_embd=2048, ffn=5632,
                 max_code=3)
    tokens = zipf_tokens(8, 1024, 8192, 1337, cuda)
    results = []
    torch.use_deterministic_algorithms(True, warn_only=True)
    try:
        for _ in range(2):
            model = make_model(cuda, seed=1337, random_pressure=True, **shape)
            optimizer = torch.optim.AdamW(model.parameters(), lr=3e-4, weight_decay=0.0)
            torch.manual_seed(5)
            losses = []
            for _ in range(2):
                optimizer.zero_grad(set_to_none=True)
                with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
                    _, loss = model(tokens[:, :-1], tokens[:, 1:])
                loss.backward()
                model.ratchet_update(validate=False)
                optimizer.step()
                losses.append(float(loss))
            states = [layer.packed.clone() for layer in model.modules()
                      if isinstance(layer, DiscreteRatchetLinear)]
            results.append((losses, states, [p.detach().clone() for p in model.parameters()]))
            print(f"run losses {losses}", flush=True)
            del model, optimizer
            torch.cuda.empty_cache()
    finally:
        torch.use_deterministic_algorithms(False)
    (l0, s0, p0), (l1, s1, p1) = results
    assert l0 == l1
    assert all(torch.equal(a, b) for a, b in zip(s0, s1))
    assert all(torch.equal(a, b) for a, b in zip(p0, p1))
