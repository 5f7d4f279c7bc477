"""DiscreteRatchetLinear on the GPU: the reference's layer tests restated
(tests/test_ratchet.py), plus integer-state parity against the oracle over 100
teacher-forced training steps of one int8 ratchet linear."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch import nn

from local_ai_training.int8_matmul import grad_weight_bf16, grad_weight_bf16_x, quantize_rows
from local_ai_training.ratchet import (
    DiscreteRatchetLinear,
    audit_no_master_weights,
    pack_code_pressure,
    unpack_code_pressure,
)
from oracle import gemm as ogemm
from oracle import quant as oquant
from oracle import update as oupd

pytestmark = pytest.mark.gpu


def test_positive_gradient_clicks_code_down_and_retains_residual_pressure(cuda):
    layer = DiscreteRatchetLinear.from_reference(torch.tensor([[1.0, 1.0]]), max_code=2,
                                                 pressure_threshold=2).to(cuda)
    stats = layer.apply_normalized_gradient(torch.tensor([[1.5, 0.5]]))
    assert layer.code.tolist() == [[1, 2]]
    assert layer.pressure.tolist() == [[0, -1]]
    assert stats.negative_moves == 1 and stats.positive_moves == 0


def test_saturated_outward_click_is_consumed_and_recorded(cuda):
    layer = DiscreteRatchetLinear.from_reference(torch.tensor([[1.0]]), max_code=2,
                                                 pressure_threshold=2).to(cuda)
    stats = layer.apply_normalized_gradient(torch.tensor([[-2.0]]))
    assert layer.code.item() == 2 and layer.pressure.item() == 0
    assert stats.blocked_positive_moves == 1 and stats.positive_moves == 0


@pytest.mark.parametrize("max_code, code_sum, pressure_sum, total_moves",
                         [(2, 15, -32, 59), (3, 14, -32, 62), (4, 9, -32, 65)])
def test_update_matches_golden_reference(cuda, max_code, code_sum, pressure_sum, total_moves):
    # tests/test_ratchet.py:196-208, on the HIP update kernel.
    torch.manual_seed(1234)
    layer = DiscreteRatchetLinear(8, 6, max_code=max_code, pressure_threshold=8).to(cuda)
    total = 0
    for _ in range(60):
        total += layer.apply_normalized_gradient(torch.randn(6, 8) * 2.0).code_moves
    assert int(layer.code.sum()) == code_sum
    assert int(layer.pressure.sum()) == pressure_sum
    assert int(total) == total_moves


def test_stored_pressure_stays_within_nibble_under_adversarial_updates(cuda):
    torch.manual_seed(0)
    for max_code in (2, 3, 4):
        for threshold in (1, 2, 4, 8):
            layer = DiscreteRatchetLinear(8, 6, max_code=max_code,
                                          pressure_threshold=threshold).to(cuda)
            for step in range(100):
                sign = 1.0 if step % 7 < 5 else -1.0
                layer.apply_normalized_gradient(sign * (3.0 + torch.rand(6, 8)), validate=False)
            assert int(layer.pressure.abs().max()) <= 7
            assert int(layer.code.abs().max()) <= max_code


def test_row_rms_normalization_is_finite_for_zero_gradient(cuda):
    layer = DiscreteRatchetLinear(4, 2, max_code=3).to(cuda)
    stats = layer.apply_weight_gradient(torch.zeros(2, 4, device=cuda))
    assert stats.code_moves == 0
    assert torch.count_nonzero(layer.pressure).item() == 0
    assert math.isfinite(stats.gradient_rms_mean)


def test_training_forward_keeps_temporary_weight_until_update_then_releases_it(cuda):
    layer = DiscreteRatchetLinear.from_reference(torch.eye(2), max_code=2).to(cuda).train()
    inputs = torch.ones(1, 2, device=cuda, requires_grad=True)
    layer(inputs).sum().backward()
    assert layer.has_pending_gradient
    stats = layer.ratchet_update()
    assert stats.total_weights == 4
    assert not layer.has_pending_gradient and layer._effective_weight is None


def test_apply_weight_gradient_rejects_nonfinite_when_validating(cuda):
    layer = DiscreteRatchetLinear(4, 2, max_code=2).to(cuda)
    g = torch.zeros(2, 4, device=cuda)
    g[0, 1] = float("nan")
    with pytest.raises(FloatingPointError):
        layer.apply_weight_gradient(g)


@pytest.mark.parametrize("mode", ["bf16", "int8"])
def test_opt_in_matmul_modes_capture_effective_gradient_and_clear(cuda, mode):
    torch.manual_seed(2)
    layer = DiscreteRatchetLinear(35, 53, max_code=3, matmul_mode=mode).to(cuda).train()
    inputs = torch.randn(2, 3, 35, device=cuda, requires_grad=True)
    output = layer(inputs)
    assert output.shape == (2, 3, 53)
    output.sum().backward()
    assert layer.has_pending_gradient
    assert layer._pending_weight_gradient.shape == (53, 35)
    assert torch.isfinite(layer._pending_weight_gradient).all()
    output2 = layer(inputs)
    with pytest.raises(RuntimeError, match="missing ratchet_update"):
        output2.sum().backward()
    layer.ratchet_update()
    layer(inputs).sum().backward()
    layer.discard_pending_gradient()
    assert not layer.has_pending_gradient


def test_bf16_mode_matches_eager_bf16_forward_and_effective_gradient(cuda):
    torch.manual_seed(4)
    layer = DiscreteRatchetLinear(17, 11, max_code=2, matmul_mode="bf16").to(cuda).train()
    inputs = torch.randn(7, 17, device=cuda, requires_grad=True)
    ref_in = inputs.detach().clone().requires_grad_(True)
    ref_w = layer.effective_weight().to(torch.bfloat16).detach().requires_grad_(True)
    expected = torch.nn.functional.linear(ref_in.to(torch.bfloat16), ref_w)
    expected.float().square().mean().backward()
    actual = layer(inputs)
    actual.float().square().mean().backward()
    assert torch.equal(actual, expected.to(actual.dtype))
    assert torch.equal(inputs.grad, ref_in.grad)
    assert torch.equal(layer._pending_weight_gradient, ref_w.grad.float())


def test_trainable_scale_gradient_matches_eager_bf16_autograd(cuda):
    torch.manual_seed(5)
    layer = DiscreteRatchetLinear(13, 9, max_code=4, matmul_mode="bf16",
                                  trainable_scale=True).to(cuda).train()
    inputs = torch.randn(6, 13, device=cuda)
    code = layer.code.float()
    ref_log = layer.log_scale.detach().clone().requires_grad_(True)
    ref_w = (code * ref_log.exp()[:, None]).to(torch.bfloat16)
    torch.nn.functional.linear(inputs.to(torch.bfloat16), ref_w).float().square().mean().backward()
    layer(inputs).float().square().mean().backward()
    assert torch.allclose(layer.log_scale.grad, ref_log.grad, atol=2e-4, rtol=2e-2)


def test_int8_mode_forward_matches_integer_reference(cuda):
    torch.manual_seed(6)
    layer = DiscreteRatchetLinear(35, 53, max_code=4, matmul_mode="int8").to(cuda).eval()
    inputs = torch.randn(2, 3, 35, device=cuda)
    q, s = quantize_rows(inputs.flatten(0, -2))
    expected = ((q.float() @ layer.code.t().float()) * s[:, None]
                * layer.scale[None, :]).to(torch.bfloat16)
    assert torch.equal(layer(inputs), expected.reshape(2, 3, 53).float())


def test_int8_effective_weight_gradient_stays_close_to_eager_autograd(cuda):
    torch.manual_seed(7)
    layer = DiscreteRatchetLinear(35, 53, max_code=3, matmul_mode="int8").to(cuda).train()
    inputs = torch.randn(67, 35, device=cuda, requires_grad=True)
    ref_w = layer.effective_weight().detach().requires_grad_(True)
    torch.nn.functional.linear(inputs.detach(), ref_w).float().square().mean().backward()
    layer(inputs).float().square().mean().backward()
    rel = (layer._pending_weight_gradient - ref_w.grad).norm() / ref_w.grad.norm()
    assert rel < 0.03


def test_int8_backward_grad_input_matches_bf16_within_tolerance(cuda):
    torch.manual_seed(11)
    weight = torch.randn(48, 32, device=cuda)
    common = dict(max_code=2, matmul_mode="int8", fuse_backward_update=True,
                  initial_weight=weight)
    bf16_bwd = DiscreteRatchetLinear(32, 48, **common).to(cuda).train()
    int8_bwd = DiscreteRatchetLinear(32, 48, int8_backward=True, **common).to(cuda).train()
    inputs = torch.randn(40, 32, device=cuda)
    q, s = quantize_rows(inputs)
    in_a = inputs.detach().clone().requires_grad_(True)
    in_b = inputs.detach().clone().requires_grad_(True)
    out_a = bf16_bwd(in_a, inputs_int8=q, inputs_scale=s)
    out_b = int8_bwd(in_b, inputs_int8=q, inputs_scale=s)
    assert torch.equal(out_a, out_b)
    grad_out = torch.randn_like(out_a)
    out_a.backward(grad_out)
    out_b.backward(grad_out)
    rel = (in_b.grad - in_a.grad).norm() / in_a.grad.norm()
    assert rel < 0.03, f"int8 grad_input relerr {rel:.4f} exceeds 0.03"
    assert torch.equal(int8_bwd.packed, bf16_bwd.packed)


@pytest.mark.parametrize("max_code", [2, 3, 4])
@pytest.mark.parametrize("trainable_scale", [False, True])
@pytest.mark.parametrize("matmul_mode", ["fp32", "bf16", "int8"])
def test_fused_backward_equivalence(cuda, max_code, trainable_scale, matmul_mode):
    torch.manual_seed(42)
    inputs = torch.randn(5, 7, 16, device=cuda, requires_grad=True)
    weight = torch.randn(32, 16, device=cuda)
    kw = dict(max_code=max_code, trainable_scale=trainable_scale, matmul_mode=matmul_mode,
              initial_weight=weight)
    eager = DiscreteRatchetLinear(16, 32, fuse_backward_update=False, **kw).to(cuda).train()
    fused = DiscreteRatchetLinear(16, 32, fuse_backward_update=True, tile_size=11,
                                  **kw).to(cuda).train()
    xe = inputs.detach().clone().requires_grad_()
    xf = inputs.detach().clone().requires_grad_()
    out_e, out_f = eager(xe), fused(xf)
    grad_out = torch.randn_like(out_e)
    out_e.backward(grad_out)
    out_f.backward(grad_out)
    se, sf = eager.ratchet_update(), fused.ratchet_update()
    assert sf.total_weights == se.total_weights
    assert (sf.positive_moves, sf.negative_moves) == (se.positive_moves, se.negative_moves)
    assert (sf.blocked_positive_moves, sf.blocked_negative_moves) == \
        (se.blocked_positive_moves, se.blocked_negative_moves)
    assert abs(sf.gradient_rms_mean - se.gradient_rms_mean) <= 1e-4 + 1e-4 * abs(se.gradient_rms_mean)
    assert torch.equal(fused.packed, eager.packed)
    if trainable_scale:
        assert torch.allclose(fused.log_scale.grad, eager.log_scale.grad, rtol=1e-4, atol=1e-4)


def test_fused_nonfinite_gradient_raises_at_validating_update(cuda):
    layer = DiscreteRatchetLinear(16, 8, max_code=2, matmul_mode="int8",
                                  fuse_backward_update=True).to(cuda).train()
    x = torch.randn(4, 16, device=cuda, requires_grad=True)
    out = layer(x)
    g = torch.randn_like(out)
    g[1, 3] = float("inf")
    out.backward(g)
    with pytest.raises(FloatingPointError):
        layer.ratchet_update(validate=True)


def test_rms_ema_beta_zero_matches_instantaneous_normalization(cuda):
    torch.manual_seed(0)
    ref = torch.randn(6, 8)
    base = DiscreteRatchetLinear(8, 6, max_code=2, initial_weight=ref.clone()).to(cuda)
    ema = DiscreteRatchetLinear(8, 6, max_code=2, rms_ema_beta=0.0,
                                initial_weight=ref.clone()).to(cuda)
    grad = torch.randn(6, 8, device=cuda)
    assert torch.equal(base._normalize(grad, 0, 6), ema._normalize(grad, 0, 6))


def test_rms_ema_first_step_matches_instantaneous_then_smooths(cuda):
    torch.manual_seed(0)
    layer = DiscreteRatchetLinear(8, 6, max_code=2, rms_ema_beta=0.9).to(cuda)
    g1 = torch.randn(6, 8, device=cuda)
    rms1 = g1.square().mean(dim=1, keepdim=True).sqrt()
    assert torch.allclose(layer._normalize(g1, 0, 6), g1 / (rms1 + layer.eps))
    g2 = torch.randn(6, 8, device=cuda) * 5.0
    ms1, ms2 = g1.square().mean(dim=1), g2.square().mean(dim=1)
    expected = g2 / ((0.9 * ms1 + 0.1 * ms2).unsqueeze(1).sqrt() + layer.eps)
    assert torch.allclose(layer._normalize(g2, 0, 6), expected)


def _force_pressure(layer, value):
    code, _ = unpack_code_pressure(layer.packed, layer.max_code)
    layer.packed.copy_(pack_code_pressure(code, torch.full_like(code, value), layer.max_code))


def test_pressure_leak_cadence_and_direction(cuda):
    layer = DiscreteRatchetLinear(8, 4, max_code=2, pressure_leak_period=0).to(cuda)
    _force_pressure(layer, 5)
    for _ in range(10):
        layer._maybe_leak_pressure()
    assert int(layer.pressure.min()) == 5 and int(layer.pressure.max()) == 5
    layer = DiscreteRatchetLinear(8, 4, max_code=2, pressure_leak_period=3).to(cuda)
    _force_pressure(layer, 5)
    for _ in range(3):
        layer._maybe_leak_pressure()
    assert int(layer.pressure.max()) == 4
    layer = DiscreteRatchetLinear(8, 4, max_code=2, pressure_leak_period=1).to(cuda)
    _force_pressure(layer, -2)
    layer._maybe_leak_pressure()
    assert int(layer.pressure.min()) == -1
    layer._validate_state()


def test_deferred_stats_materialize_equals_eager_item(cuda):
    torch.manual_seed(0)
    layer = DiscreteRatchetLinear(16, 8, max_code=2).to(cuda)
    grad = torch.randn(8, 16, device=cuda)
    normalized = grad / (grad.square().mean(dim=1, keepdim=True).sqrt() + 1e-8)
    stats = layer.apply_normalized_gradient(normalized.clone(), validate=False)
    assert isinstance(stats.positive_moves, torch.Tensor)
    m = stats.materialize()
    assert isinstance(m.positive_moves, int)
    assert m.positive_moves == int(stats.positive_moves.item())
    assert m.code_moves == m.positive_moves + m.negative_moves
    assert m.total_weights == 8 * 16


def test_trainable_scale_receives_gradient_and_stays_master_weight_free(cuda):
    torch.manual_seed(0)
    layer = DiscreteRatchetLinear(4, 3, max_code=2, trainable_scale=True).to(cuda).train()
    assert audit_no_master_weights(nn.Sequential(layer)).violations == ()
    optimizer = torch.optim.AdamW(layer.parameters(), lr=0.1)
    before = layer.scale.detach().clone()
    layer(torch.randn(5, 4, device=cuda)).square().mean().backward()
    assert layer.log_scale.grad is not None
    layer.ratchet_update()
    optimizer.step()
    assert not torch.equal(layer.scale.detach(), before) and torch.all(layer.scale > 0)


def test_float32_gradient_grad_weight_from_the_quant_pass_bf16_copy(cuda):
    """A float32 upstream gradient reaches grad_weight as the bf16 copy the SR-quant pass
    writes; the update must receive exactly what the grad_weight kernel gives when it
    converts the float32 gradient itself (both round to nearest even)."""
    m, k, n = 1024, 512, 768
    torch.manual_seed(5)
    layer = DiscreteRatchetLinear(k, n, max_code=2, matmul_mode="int8", int8_backward=True,
                                  fuse_backward_update=True).to(cuda).train()
    layer.keep_weight_gradient = True  # the bf16 gradient the fused update consumed
    data = torch.Generator().manual_seed(8)
    x = torch.randn(m, k, generator=data).to(cuda)
    g = (torch.randn(m, n, generator=data) * 1e-2).to(cuda)
    q, s = quantize_rows(x)
    out = layer(x.clone().requires_grad_(True), inputs_int8=q, inputs_scale=s)
    assert out.dtype == torch.float32
    out.backward(g)
    want = grad_weight_bf16(g, q, s)
    assert torch.equal(layer.last_weight_gradient.view(torch.int16), want.view(torch.int16))


def test_unfused_int8_layer_grad_weight_reads_the_saved_inputs(cuda):
    """Without pre-quantized inputs (the lm_head case) grad_weight is bf16(g)^T @ bf16(x)
    on the saved float32 inputs (ratchet.py:159-163); the update must receive exactly the
    direct-activation kernel's result, which matches an fp32 product of the same bf16
    operands at rel 1e-2 / abs 1e-3."""
    m, k, n = 2048, 512, 1024
    torch.manual_seed(6)
    layer = DiscreteRatchetLinear(k, n, max_code=2, matmul_mode="int8",
                                  fuse_backward_update=True).to(cuda).train()
    layer.keep_weight_gradient = True
    data = torch.Generator().manual_seed(9)
    x = torch.randn(m, k, generator=data).to(cuda)
    g = torch.randn(m, n, generator=data).to(cuda) * 1e-2
    out = layer(x.clone().requires_grad_(True))
    out.backward(g)
    want = grad_weight_bf16_x(g.to(torch.bfloat16), x)
    assert torch.equal(layer.last_weight_gradient.view(torch.int16), want.view(torch.int16))
    ref = g.to(torch.bfloat16).float().t() @ x.to(torch.bfloat16).float()
    got = layer.last_weight_gradient.float()
    assert bool(((got - ref).abs() <= 1e-3 + 1e-2 * ref.abs()).all())


def test_hundred_step_integer_state_parity_with_shared_grad_weight(cuda):
    """100 int8 training steps of one ratchet linear (int8 fwd, int8 SR grad_input, bf16
    grad_weight, fused update). Each step the oracle recomputes, from the same inputs and
    the same SR seed, the forward output, the SR-quantized gradient and grad_input, and
    applies the update to its own packed copy using the grad_weight the GPU produced
    (the one float producer shared, since BLAS reductions are not reproducible). Forward
    output, grad_input and the packed state must stay bit-identical every step."""
    m, k, n, mc = 512, 256, 384, 2
    torch.manual_seed(1337)
    layer = DiscreteRatchetLinear(k, n, max_code=mc, matmul_mode="int8", int8_backward=True,
                                  fuse_backward_update=True).to(cuda).train()
    packed_ref = layer.packed.cpu().numpy().copy()
    scale = layer.scale.float().cpu().numpy()
    # the weight gradient the fused update consumes (the one float producer shared with
    # the oracle), kept by the update itself
    layer.keep_weight_gradient = True
    data = torch.Generator().manual_seed(99)
    for step in range(100):
        x = torch.randn(m, k, generator=data).to(torch.bfloat16)
        gout = (torch.randn(m, n, generator=data) * 1e-2).to(torch.bfloat16)
        xd = x.to(cuda).requires_grad_(True)
        q, s = quantize_rows(xd.detach())
        out = layer(xd, inputs_int8=q, inputs_scale=s)
        rng_state = torch.get_rng_state()
        out.backward(gout.to(cuda))
        stats = layer.ratchet_update(validate=False)
        # oracle replay
        q_ref, s_ref = oquant.quantize_rows(x.float().numpy())
        code, _ = oupd.unpack(packed_ref, mc)
        out_ref = ogemm.scaled_int8_mm(q_ref, code.T, s_ref, scale)
        assert np.array_equal(out.detach().to(torch.bfloat16).cpu().view(torch.int16).numpy()
                              .view(np.uint16), out_ref), f"forward differs at step {step}"
        torch.set_rng_state(rng_state)
        seed = int(torch.randint(0, 2**31 - 1, (1,)).item())
        gq, gs = oquant.quantize_rows_sr(gout.float().numpy(), scale, seed)
        gin_ref = ogemm.scaled_int8_mm(gq, code, gs, None)
        gin = xd.grad.to(torch.bfloat16).cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(gin, gin_ref), f"grad_input differs at step {step}"
        gw = layer.last_weight_gradient
        assert gw.dtype == torch.bfloat16
        # grad_weight = bf16(g)^T @ bf16(x_hat) in fp32, bf16 output: rel 1e-2 / abs 1e-3.
        xh = (torch.from_numpy(q_ref).to(torch.bfloat16)
              * torch.from_numpy(s_ref).to(torch.bfloat16)[:, None]).float()
        gw_ref = gout.float().t() @ xh
        torch.testing.assert_close(gw.float().cpu(), gw_ref, rtol=1e-2, atol=1e-3)
        ref = oupd.update_from_gradient(packed_ref, gw.float().cpu().numpy(), mc, 8, 0.5, 1.5,
                                        1e-8, oupd.vec_for_dtype("bf16"))
        packed_ref = ref["packed"]
        assert np.array_equal(layer.packed.cpu().numpy(), packed_ref), f"state differs at {step}"
        m_stats = stats.materialize()
        assert [m_stats.positive_moves, m_stats.negative_moves, m_stats.blocked_positive_moves,
                m_stats.blocked_negative_moves] == ref["counts"].tolist()
    c, p = oupd.unpack(packed_ref, mc)
    assert np.abs(p).max() <= 7 and np.abs(c).max() <= mc


def test_int8_out_dtype_override_gives_the_same_values_and_update(cuda):
    # out_dtype=bf16 hands over the GEMM's bf16 result; the default float32 output is that
    # result widened. Forward values, grad_input and the updated state are identical when
    # the gradient is the same (bf16-exact) values in either dtype.
    m, k, n, mc = 512, 256, 384, 2
    layers = []
    for _ in range(2):
        torch.manual_seed(11)
        layers.append(DiscreteRatchetLinear(k, n, max_code=mc, matmul_mode="int8",
                                            int8_backward=True,
                                            fuse_backward_update=True).to(cuda).train())
    torch.manual_seed(12)
    x = torch.randn(m, k, device=cuda)
    g = (torch.randn(m, n, device=cuda) * 1e-2).to(torch.bfloat16)
    q, s = quantize_rows(x)
    start = layers[0].packed.clone()
    outs, grads = [], []
    for layer, dt in zip(layers, (None, torch.bfloat16)):
        xi = x.clone().requires_grad_(True)
        out = layer(xi, inputs_int8=q, inputs_scale=s, out_dtype=dt)
        torch.manual_seed(13)  # the SR seed is drawn from the host RNG in backward
        out.backward(g.float() if dt is None else g)
        layer.ratchet_update(validate=True)
        outs.append(out)
        grads.append(xi.grad)
    assert outs[0].dtype == torch.float32 and outs[1].dtype == torch.bfloat16
    assert torch.equal(outs[1].float(), outs[0])
    assert torch.equal(grads[0], grads[1])
    assert torch.equal(layers[0].packed, layers[1].packed)
    assert not torch.equal(layers[0].packed, start)  # the update did move pressure


def test_int8_residual_argument_matches_adding_afterwards(cuda):
    # residual= on an int8 layer: a full-shape float32 residual goes through the GEMM's
    # epilogue, a broadcast [n] one through the separate add. Values, the residual's gradient
    # (summed to its shape), grad_input and the updated state equal those of adding after.
    m, k, n, mc = 512, 256, 384, 2
    torch.manual_seed(12)
    x = torch.randn(m, k, device=cuda)
    g = torch.randn(m, n, device=cuda) * 1e-2
    q, s = quantize_rows(x)
    for shape in ((m, n), (n,)):
        r0 = torch.randn(*shape, device=cuda)
        results = []
        for fused in (True, False):
            torch.manual_seed(11)
            layer = DiscreteRatchetLinear(k, n, max_code=mc, matmul_mode="int8",
                                          int8_backward=True,
                                          fuse_backward_update=True).to(cuda).train()
            xi = x.clone().requires_grad_(True)
            r = r0.clone().requires_grad_(True)
            if fused:
                out = layer(xi, inputs_int8=q, inputs_scale=s, residual=r)
            else:
                out = r + layer(xi, inputs_int8=q, inputs_scale=s)
            torch.manual_seed(13)  # the SR seed is drawn from the host RNG in backward
            out.backward(g)
            layer.ratchet_update(validate=True)
            results.append((out.detach(), xi.grad, r.grad, layer.packed.clone()))
        for a, b in zip(*results):
            assert a.shape == b.shape and torch.equal(a, b), shape
