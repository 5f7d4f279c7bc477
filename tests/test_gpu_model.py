"""The ratchet GPT on the GPU: forward/backward/fused update in every matmul mode,
and the fused int8 prologues against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from local_ai_training.int8_fused import (
    fused_gelu_quantize,
    fused_rmsnorm_quantize,
    fused_transpose_quantize,
)
from local_ai_training.model import ModelConfig, build_seeded_model
from local_ai_training.ratchet import DiscreteRatchetLinear
from oracle import quant as oquant

pytestmark = pytest.mark.gpu


def tiny_config(**kw) -> ModelConfig:
    return ModelConfig(vocab_size=11, block_size=8, n_layer=2, n_head=2, n_embd=16, **kw)


@pytest.mark.parametrize("mode,int8_backward", [("fp32", False), ("bf16", False),
                                                ("int8", False), ("int8", True)])
def test_forward_backward_and_ratchet_update_clear_all_temporary_weights(cuda, mode,
                                                                        int8_backward):
    # tests/test_model.py:42-56 in each matmul mode.
    config = tiny_config(matmul_mode=mode, int8_backward=int8_backward)
    model = build_seeded_model(config, max_code=3, seed=5).to(cuda).train()
    tokens = torch.randint(0, config.vocab_size, (3, config.block_size)).to(cuda)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        logits, loss = model(tokens, tokens)
    assert logits.shape == (3, config.block_size, config.vocab_size)
    assert torch.isfinite(loss)
    loss.backward()
    stats = model.ratchet_update()
    layers = [m for m in model.modules() if isinstance(m, DiscreteRatchetLinear)]
    assert stats.total_weights == sum(layer.packed.numel() for layer in layers)
    assert all(not layer.has_pending_gradient for layer in layers)
    for layer in layers:
        assert int(layer.code.abs().max()) <= 3 and int(layer.pressure.abs().max()) <= 7


def test_int8_training_moves_codes_and_lowers_loss(cuda):
    torch.manual_seed(0)
    config = ModelConfig(vocab_size=16, block_size=32, n_layer=2, n_head=4, n_embd=64,
                         matmul_mode="int8", int8_backward=True)
    model = build_seeded_model(config, max_code=2, seed=1337).to(cuda).train()
    optimizer = torch.optim.AdamW(model.parameters(), lr=3e-3, weight_decay=0.0)
    pattern = torch.arange(33) % 4  # a learnable periodic sequence
    batch = torch.stack([torch.roll(pattern, s) for s in range(16)]).to(cuda)
    inputs, targets = batch[:, :32], batch[:, 1:]
    losses, moves = [], 0
    for _ in range(60):
        optimizer.zero_grad(set_to_none=True)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            _, loss = model(inputs, targets)
        loss.backward()
        stats = model.ratchet_update(validate=False)
        optimizer.step()
        losses.append(float(loss))
        moves += int(stats.code_moves)
    assert moves > 0
    assert np.mean(losses[-10:]) < np.mean(losses[:10]) - 0.1


def _rms_norm_f64(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)


def _gelu_tanh_f64(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float64)
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def _assert_quant_close(q, s, y_ref):
    # Transcendentals / reduction order make the float transform differ in the last ulp,
    # so codes on a rounding boundary may differ by one (the reference's own fused
    # prologues are only checked against torch ops the same way).
    q_ref, s_ref = oquant.quantize_rows(y_ref.astype(np.float32))
    q = q.cpu().numpy().reshape(q_ref.shape)
    s = s.cpu().numpy().reshape(s_ref.shape)
    assert np.allclose(s, s_ref, rtol=1e-5, atol=0)
    diff = np.abs(q.astype(np.int32) - q_ref.astype(np.int32))
    assert diff.max() <= 1
    assert (diff > 0).mean() < 1e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(33, 64), (1024, 512), (7, 2048)])
def test_fused_rmsnorm_quantize(cuda, shape, dtype):
    g = torch.Generator().manual_seed(shape[0])
    x = (torch.randn(shape, generator=g) * 2.0).to(dtype)
    w = torch.rand(shape[1], generator=g) + 0.5
    q, s = fused_rmsnorm_quantize(x.to(cuda), w.to(cuda), 1e-5)
    _assert_quant_close(q, s, _rms_norm_f64(x.float().numpy(), w.numpy(), 1e-5))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(33, 64), (1024, 2048)])
def test_fused_gelu_quantize(cuda, shape, dtype):
    x = (torch.randn(shape, generator=torch.Generator().manual_seed(3)) * 2.0).to(dtype)
    q, s = fused_gelu_quantize(x.to(cuda))
    _assert_quant_close(q, s, _gelu_tanh_f64(x.float().numpy()))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_transpose_quantize_is_exact(cuda, dtype):
    b, h, s_len, d = 3, 4, 10, 16
    x = torch.randn(b, h, s_len, d, generator=torch.Generator().manual_seed(4)).to(dtype)
    q, s = fused_transpose_quantize(x.to(cuda))
    rows = x.transpose(1, 2).reshape(b * s_len, h * d).float().numpy()
    q_ref, s_ref = oquant.quantize_rows(rows)
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)
    # a strided (non-contiguous) producer layout
    xt = x.to(cuda).transpose(2, 3).contiguous().transpose(2, 3)
    q2, s2 = fused_transpose_quantize(xt)
    assert torch.equal(q2.cpu(), q.cpu()) and torch.equal(s2.cpu(), s.cpu())


def _int8_steps(cuda, fuse: bool, steps: int = 3, bf16_expand: bool = True,
                fuse_grad: bool = True, split_qkv: bool = True):
    from local_ai_training.model import CausalSelfAttention, FeedForward, TransformerBlock

    TransformerBlock.fuse_residual = fuse
    TransformerBlock.fuse_residual_grad = fuse_grad
    FeedForward.bf16_expand = bf16_expand
    CausalSelfAttention.split_qkv_grad = split_qkv
    try:
        torch.manual_seed(0)
        config = ModelConfig(vocab_size=64, block_size=64, n_layer=2, n_head=4, n_embd=128,
                             matmul_mode="int8", int8_backward=True)
        model = build_seeded_model(config, max_code=2, seed=1337).to(cuda).train()
        optimizer = torch.optim.AdamW(model.parameters(), lr=3e-3, weight_decay=0.0)
        gen = torch.Generator().manual_seed(3)
        batch = torch.randint(0, 64, (8, 65), generator=gen).to(cuda)
        losses = []
        for _ in range(steps):
            optimizer.zero_grad(set_to_none=True)
            with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
                _, loss = model(batch[:, :64], batch[:, 1:])
            loss.backward()
            model.ratchet_update(validate=True)
            optimizer.step()
            losses.append(loss.detach())
        states = [m.packed.clone() for m in model.modules() if isinstance(m, DiscreteRatchetLinear)]
        params = [p.detach().clone() for p in model.parameters()]
        return losses, states, params
    finally:
        TransformerBlock.fuse_residual = True
        TransformerBlock.fuse_residual_grad = True
        FeedForward.bf16_expand = True
        CausalSelfAttention.split_qkv_grad = True


def test_residual_fused_into_the_gemm_epilogue_changes_nothing(cuda):
    # The residual stream added by the projection / contraction GEMMs' epilogue instead of a
    # separate add: identical losses, ratchet states and float parameters over three steps.
    from local_ai_training import ratchet

    calls = []
    fused_mm = ratchet.packed_int8_mm_residual

    def counting(*args, **kwargs):
        calls.append(1)
        return fused_mm(*args, **kwargs)

    ratchet.packed_int8_mm_residual = counting
    try:
        la, sa, pa = _int8_steps(cuda, fuse=True)
    finally:
        ratchet.packed_int8_mm_residual = fused_mm
    assert len(calls) == 3 * 2 * 2  # steps x layers x (projection, contraction)
    lb, sb, pb = _int8_steps(cuda, fuse=False)
    assert torch.equal(la[0], lb[0])  # forward
    assert all(torch.equal(x, y) for x, y in zip(la, lb))
    assert all(torch.equal(x, y) for x, y in zip(sa, sb))
    assert all(torch.equal(x, y) for x, y in zip(pa, pb))


@pytest.mark.parametrize("fuse", [True, False])
def test_bf16_expansion_hand_off_changes_nothing(cuda, fuse):
    # Under bf16 autocast the expansion hands its bf16 GEMM result to the GELU prologue
    # instead of the float32 widening of it: the GELU quant, the contraction's bf16
    # grad_input, the GELU backward's bf16-rounded gradient and the expansion's SR quant and
    # grad_weight see the same values, so losses, ratchet states and float parameters are
    # identical over three steps (with the residual added in the epilogue and separately).
    from local_ai_training import int8_backward

    seen = []
    gelu_bwd = int8_backward.gelu_backward

    def recording(grad_y, x):
        seen.append((grad_y.dtype, x.dtype))
        return gelu_bwd(grad_y, x)

    int8_backward.gelu_backward = recording
    try:
        la, sa, pa = _int8_steps(cuda, fuse=fuse, bf16_expand=True)
    finally:
        int8_backward.gelu_backward = gelu_bwd
    assert seen and all(d == (torch.bfloat16, torch.bfloat16) for d in seen)
    lb, sb, pb = _int8_steps(cuda, fuse=fuse, bf16_expand=False)
    assert all(torch.equal(x, y) for x, y in zip(la, lb))
    assert all(torch.equal(x, y) for x, y in zip(sa, sb))
    assert all(torch.equal(x, y) for x, y in zip(pa, pb))


def test_residual_gradient_added_in_the_rmsnorm_backward_changes_nothing(cuda):
    # The block input's gradient from the residual stream added in the RMSNorm backward's
    # store (FusedRMSNormQuantizeResidualFn) instead of by autograd: identical losses,
    # ratchet states and float parameters over three steps, and no separate add runs.
    from local_ai_training import int8_backward

    calls = []
    orig = int8_backward.rmsnorm_backward

    def recording(*args, **kwargs):
        calls.append(kwargs.get("residual_grad") is not None)
        return orig(*args, **kwargs)

    int8_backward.rmsnorm_backward = recording
    try:
        la, sa, pa = _int8_steps(cuda, fuse=True, fuse_grad=True)
    finally:
        int8_backward.rmsnorm_backward = orig
    assert calls and all(calls)
    lb, sb, pb = _int8_steps(cuda, fuse=True, fuse_grad=False)
    assert all(torch.equal(x, y) for x, y in zip(la, lb))
    assert all(torch.equal(x, y) for x, y in zip(sa, sb))
    assert all(torch.equal(x, y) for x, y in zip(pa, pb))


def test_qkv_gradients_read_in_parts_change_nothing(cuda):
    # The qkv layer returning q, k, v itself, so that its backward quantizes dq, dk, dv and
    # forms the weight gradient from them in place instead of from their concatenation:
    # identical losses, ratchet states and float parameters over three steps.
    from local_ai_training import ratchet

    calls = []
    cls = ratchet._RatchetMatmul
    orig = cls.__dict__["_backward_parts"]

    def recording(*args, **kwargs):
        calls.append(1)
        return orig.__func__(*args, **kwargs)

    cls._backward_parts = staticmethod(recording)
    try:
        la, sa, pa = _int8_steps(cuda, fuse=True, split_qkv=True)
    finally:
        cls._backward_parts = orig
    assert len(calls) == 3 * 2  # both layers' qkv, every step
    lb, sb, pb = _int8_steps(cuda, fuse=True, split_qkv=False)
    assert all(torch.equal(x, y) for x, y in zip(la, lb))
    assert all(torch.equal(x, y) for x, y in zip(sa, sb))
    assert all(torch.equal(x, y) for x, y in zip(pa, pb))


def test_shared_move_count_buffer_gives_the_per_layer_totals(cuda):
    # The model's one [layers, 4] move-count buffer (summed and cleared once per step) gives
    # the same step statistics as per-layer count tensors, step after step, and a
    # layer-level ratchet_update in between (which leaves its slot to be cleared before its
    # next use) does not leak counts into the next step. The same for the row-rms buffer
    # whose per-layer means one launch takes: gradient_rms_mean equal bit for bit, also
    # for a layer-level ratchet_update (its own mean launch) and for a step with two
    # backward passes (the second launch of each layer keeps its own row rms).
    from local_ai_training.model import RatchetGPT

    def run(shared: bool):
        RatchetGPT.shared_move_counts = shared
        try:
            torch.manual_seed(0)
            config = ModelConfig(vocab_size=64, block_size=64, n_layer=2, n_head=4, n_embd=128,
                                 matmul_mode="int8", int8_backward=True)
            model = build_seeded_model(config, max_code=2, seed=1337).to(cuda).train()
            gen = torch.Generator().manual_seed(3)
            batch = torch.randint(0, 64, (8, 65), generator=gen).to(cuda)
            out = []
            for step in range(5):
                for _ in range(2 if step == 3 else 1):
                    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
                        _, loss = model(batch[:, :64], batch[:, 1:])
                    loss.backward()
                if step == 2:
                    first = next(m for m in model.modules()
                                 if isinstance(m, DiscreteRatchetLinear))
                    out.append(first.ratchet_update(validate=True))
                out.append(model.ratchet_update(validate=True))
            return out
        finally:
            RatchetGPT.shared_move_counts = True

    shared, separate = run(True), run(False)
    assert shared == separate
    assert any(s.code_moves > 0 for s in shared)


def test_layer_stats_keep_their_counts_across_model_updates(cuda):
    # A layer's RatchetUpdateStats (from its own ratchet_update, counts in the model's shared
    # slot) keep their values after the model's update sums and clears that slot and the
    # next step reuses it, as the reference's per-layer stats own their tensors.
    from local_ai_training.ratchet import pack_code_pressure

    torch.manual_seed(0)
    config = ModelConfig(vocab_size=64, block_size=64, n_layer=2, n_head=4, n_embd=128,
                         matmul_mode="int8", int8_backward=True)
    model = build_seeded_model(config, max_code=2, seed=1337).to(cuda).train()
    first = next(m for m in model.modules() if isinstance(m, DiscreteRatchetLinear))
    gen = torch.Generator().manual_seed(4)
    near = (torch.randint(0, 2, tuple(first.packed.shape), generator=gen,
                          dtype=torch.int8) * 14 - 7)
    first.packed.copy_(pack_code_pressure(first.code.cpu(), near, 2).to(cuda))
    batch = torch.randint(0, 64, (8, 65), generator=gen).to(cuda)

    def step():
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            _, loss = model(batch[:, :64], batch[:, 1:])
        loss.backward()

    step()
    kept = first.ratchet_update(validate=True)
    fields = ("positive_moves", "negative_moves", "blocked_positive_moves",
              "blocked_negative_moves")
    before = [int(getattr(kept, f)) for f in fields]
    model.ratchet_update(validate=True)
    step()
    model.ratchet_update(validate=True)
    torch.cuda.synchronize()
    assert [int(getattr(kept, f)) for f in fields] == before
    assert sum(before) > 0
