"""The HIP cross-entropy (``local_ai_training.cross_entropy``) against the loss it replaces,
``F.cross_entropy(logits, targets)`` (reference ``model.py:249``, mean reduction,
``ignore_index``).

Checked against torch's CPU loss and gradient in float64 on the same logits (the
mathematical values; our float32 arithmetic must land within its rounding), and against
torch's own float32 GPU loss, whose gradient rounded to bfloat16 must match ours to one
bfloat16 step. The training-step shapes are the 25M (16384 x 8192) and 1B (8192 x 8192)
logits; edge cases: ignored rows, all rows ignored, one row, large offsets, -inf logits.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from local_ai_training.cross_entropy import CrossEntropyFn, cross_entropy, cross_entropy_supported

pytestmark = pytest.mark.gpu


def reference(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int = -100):
    """torch's loss and logits gradient in float64 on the CPU."""
    x = logits.detach().double().cpu().requires_grad_(True)
    loss = F.cross_entropy(x, targets.cpu(), ignore_index=ignore_index)
    loss.backward()
    return loss.detach(), x.grad


def run(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int = -100,
        grad_loss: float = 1.0):
    x = logits.detach().clone().requires_grad_(True)
    loss = CrossEntropyFn.apply(x, targets, ignore_index)
    loss.backward(torch.tensor(grad_loss, device=x.device))
    return loss.detach(), x.grad


def make(m, v, dtype, cuda, seed, scale=3.0, offset=0.0):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(m, v, generator=g) * scale + offset).to(dtype).to(cuda)
    targets = torch.randint(0, v, (m,), generator=g).to(cuda)
    return logits, targets


def check_against_float64(logits, targets, loss, grad, ignore_index=-100, grad_loss=1.0):
    ref_loss, ref_grad = reference(logits, targets, ignore_index)
    ref_grad = ref_grad * grad_loss
    assert math.isclose(loss.item(), ref_loss.item(), rel_tol=1e-5, abs_tol=1e-6), \
        (loss.item(), ref_loss.item())
    got = grad.double().cpu()
    assert got.dtype == torch.float64 and got.shape == ref_grad.shape
    # float32 arithmetic (relative error ~1e-6 of each term) then one rounding to the
    # gradient's dtype: bfloat16 keeps 8 significant bits (half a step = 2^-9 relative)
    rel = 2.0 ** -8 if grad.dtype == torch.bfloat16 else 1e-5
    scale = ref_grad.abs().amax(dim=1, keepdim=True).clamp_min(1e-30)
    err = (got - ref_grad).abs()
    assert bool((err <= rel * ref_grad.abs() + 1e-6 * scale).all()), float((err / scale).max())


@pytest.mark.parametrize("m,v", [(16384, 8192), (8192, 8192)])
def test_training_shapes_bf16_against_float64(cuda, m, v):
    print(f"cross entropy bf16 {m}x{v}", flush=True)
    logits, targets = make(m, v, torch.bfloat16, cuda, seed=m + v)
    loss, grad = run(logits, targets)
    assert grad.dtype == torch.bfloat16
    check_against_float64(logits, targets, loss, grad)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,v", [(1, 8), (7, 24), (300, 1000), (64, 16384), (16, 65536)])
def test_small_and_long_rows_against_float64(cuda, dtype, m, v):
    if v % (16 // torch.empty((), dtype=dtype).element_size()):
        pytest.skip("class count not a whole number of 16-byte vectors")
    print(f"cross entropy {dtype} {m}x{v}", flush=True)
    logits, targets = make(m, v, dtype, cuda, seed=v)
    loss, grad = run(logits, targets, grad_loss=0.37)
    assert grad.dtype == dtype
    check_against_float64(logits, targets, loss, grad, grad_loss=0.37)


def test_ignored_rows_and_large_offsets(cuda):
    logits, targets = make(513, 512, torch.float32, cuda, seed=5, scale=20.0, offset=1e4)
    targets[::3] = -100
    loss, grad = run(logits, targets)
    check_against_float64(logits, targets, loss, grad)
    assert bool((grad[::3] == 0).all())
    # another ignore_index
    targets2 = targets.clone()
    targets2[::3] = 7
    targets2[1::5] = 3
    loss, grad = run(logits, targets2, ignore_index=3)
    check_against_float64(logits, targets2, loss, grad, ignore_index=3)


def test_negative_infinity_logits(cuda):
    logits, targets = make(32, 64, torch.float32, cuda, seed=6)
    logits[:, 40:] = float("-inf")
    targets = targets % 40
    loss, grad = run(logits, targets)
    ref_loss, ref_grad = reference(logits, targets)
    assert math.isclose(loss.item(), ref_loss.item(), rel_tol=1e-5)
    assert bool((grad[:, 40:] == 0).all())
    assert torch.allclose(grad[:, :40].double().cpu(), ref_grad[:, :40], rtol=1e-5, atol=1e-9)


def test_all_rows_ignored_gives_nan_like_torch(cuda):
    logits, targets = make(8, 16, torch.float32, cuda, seed=7)
    targets[:] = -100
    loss, grad = run(logits, targets)
    assert math.isnan(loss.item())
    assert math.isnan(F.cross_entropy(logits, targets).item())


def test_target_out_of_range_gives_nan_loss(cuda):
    logits, targets = make(8, 16, torch.float32, cuda, seed=8)
    targets[3] = 16
    loss, _ = run(logits, targets)
    assert math.isnan(loss.item())


def test_matches_torch_gpu_loss_and_bf16_gradient(cuda):
    """torch's float32 GPU loss on the widened bf16 logits, its gradient rounded to bf16:
    our loss within float rounding, our bf16 gradient within one bf16 step everywhere and
    equal almost everywhere."""
    logits, targets = make(4096, 8192, torch.bfloat16, cuda, seed=9)
    x = logits.float().requires_grad_(True)
    ref = F.cross_entropy(x, targets)
    ref.backward()
    ref_grad = x.grad.to(torch.bfloat16)
    loss, grad = run(logits, targets)
    assert math.isclose(loss.item(), ref.item(), rel_tol=1e-5)
    a = grad.view(torch.int16).int()
    b = ref_grad.view(torch.int16).int()
    steps = (a - b).abs()
    same_sign = (grad.float() * ref_grad.float() >= 0)
    assert bool(same_sign.all())
    assert int(steps.max()) <= 1
    assert float((steps == 0).float().mean()) > 0.999


def test_runs_repeat_bit_for_bit(cuda):
    logits, targets = make(2048, 8192, torch.bfloat16, cuda, seed=10)
    l1, g1 = run(logits, targets)
    l2, g2 = run(logits, targets)
    assert torch.equal(l1, l2) and torch.equal(g1, g2)


def test_unsupported_shapes_fall_back_to_torch(cuda):
    logits, targets = make(5, 10, torch.float32, cuda, seed=11)  # 10 % 4 != 0
    assert not cross_entropy_supported(logits, targets)
    loss = cross_entropy(logits, targets)
    assert torch.equal(loss, F.cross_entropy(logits, targets))


def test_model_loss_and_training_step_against_torch_loss(cuda):
    """A small int8 ratchet model: the fused loss (bf16 logits) against F.cross_entropy on
    the model's float32 logits, the same forward; then one training step each way from the
    same state, and the losses of the next forward agree."""
    from local_ai_training.model import ModelConfig, build_seeded_model
    from local_ai_training.training import training_step

    cfg = ModelConfig(vocab_size=256, block_size=64, n_layer=2, n_head=4, n_embd=128,
                      dropout=0.0, matmul_mode="int8", int8_backward=True)
    g = torch.Generator().manual_seed(3)
    tokens = torch.randint(0, 256, (8, 64), generator=g).to(cuda)
    targets = torch.randint(0, 256, (8, 64), generator=g).to(cuda)
    losses = {}
    for fused in (True, False):
        torch.manual_seed(0)
        model = build_seeded_model(cfg, max_code=2, seed=0).to(cuda)
        model.fused_cross_entropy = fused
        opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits, loss = model(tokens, targets)
        assert logits.dtype == (torch.bfloat16 if fused else torch.float32)
        torch.manual_seed(1)
        step_loss, _ = training_step(model, opt, tokens, targets)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            _, after = model(tokens, targets)
        losses[fused] = (loss.item(), step_loss.item(), after.item(), logits.float())
    a, b = losses[True], losses[False]
    assert torch.equal(a[3], b[3])  # the same logit values
    assert math.isclose(a[0], b[0], rel_tol=1e-5)
    assert math.isclose(a[1], b[1], rel_tol=1e-5)
    assert math.isclose(a[2], b[2], rel_tol=1e-3)
