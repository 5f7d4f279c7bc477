"""Host-side behaviour that needs no GPU: drop-in errors, construction, model configs."""

import pytest
import torch
from torch import nn

from local_ai_training.int8_matmul import (
    quantize_columns,
    quantize_rows,
    quantize_rows_colscaled,
    scaled_int8_mm,
)
from local_ai_training.model import ModelConfig, RatchetGPT, build_seeded_model
from local_ai_training.ratchet import (
    DiscreteRatchetLinear,
    audit_no_master_weights,
    bucket_pressure,
    compare_persistent_footprint,
    pack_code_pressure,
    unpack_code_pressure,
)


def test_int8_entry_points_reject_cpu_operands():
    # tests/test_int8_matmul.py:143-169: the int8 path is GPU-only.
    with pytest.raises(RuntimeError, match="CUDA"):
        quantize_rows(torch.ones(2, 3))
    with pytest.raises(RuntimeError, match="CUDA"):
        quantize_columns(torch.ones(2, 3))
    with pytest.raises(RuntimeError, match="CUDA"):
        quantize_rows_colscaled(torch.ones(2, 3), torch.ones(3))
    with pytest.raises(RuntimeError, match="requires CUDA"):
        scaled_int8_mm(torch.ones(2, 3, dtype=torch.int8), torch.ones(3, 4, dtype=torch.int8),
                       torch.ones(2), torch.ones(4))


def test_update_paths_reject_cpu_state_instead_of_falling_back():
    layer = DiscreteRatchetLinear(4, 3, max_code=2)
    with pytest.raises(RuntimeError, match="CUDA"):
        layer.apply_normalized_gradient(torch.zeros(3, 4))
    with pytest.raises(RuntimeError, match="CUDA"):
        layer.apply_weight_gradient(torch.zeros(3, 4))


def test_bucket_pressure_known_answer_via_torch(golden):
    kat = golden["bucket_pressure"]
    out = bucket_pressure(torch.tensor(kat["z"]), low=kat["low"], high=kat["high"])
    assert out.tolist() == kat["expected"]
    with pytest.raises(ValueError):
        bucket_pressure(torch.zeros(2), low=1.0, high=0.5)


@pytest.mark.parametrize("max_code", [2, 3, 4])
def test_pack_unpack_round_trip_on_cpu(max_code):
    codes = torch.arange(-max_code, max_code + 1, dtype=torch.int8)
    pressures = torch.arange(-7, 8, dtype=torch.int8)
    cg, pg = torch.meshgrid(codes, pressures, indexing="ij")
    c, p = unpack_code_pressure(pack_code_pressure(cg, pg, max_code), max_code)
    assert torch.equal(c, cg) and torch.equal(p, pg)


@pytest.mark.parametrize("max_code", [1, 2, 3, 4, 5, 6, 7])
def test_constructor_accepts_nibble_cap_and_builds_valid_state(max_code):
    layer = DiscreteRatchetLinear(8, 4, max_code=max_code)
    assert layer.packed.dtype == torch.uint8 and layer.packed.shape == (4, 8)
    assert int(layer.code.abs().max()) <= max_code
    assert int(layer.pressure.abs().max()) == 0


def test_constructor_validation_errors():
    with pytest.raises(ValueError):
        DiscreteRatchetLinear(8, 4, max_code=8)
    with pytest.raises(ValueError):
        DiscreteRatchetLinear(8, 4, max_code=2, pressure_threshold=0)
    with pytest.raises(ValueError):
        DiscreteRatchetLinear(8, 4, max_code=2, bucket_low=1.0, bucket_high=0.5)
    with pytest.raises(ValueError):
        DiscreteRatchetLinear(8, 4, max_code=2, rms_ema_beta=1.0)
    with pytest.raises(ValueError):
        DiscreteRatchetLinear(0, 4, max_code=2)


def test_buffers_and_audit_match_reference_layout():
    # tests/test_ratchet.py:250-257, 95-106, 211-221
    layer = DiscreteRatchetLinear(7, 5, max_code=2, matmul_mode="int8")
    assert dict(layer.named_parameters()) == {}
    assert set(dict(layer.named_buffers())) == {"packed", "_scale"}
    model = nn.Sequential(DiscreteRatchetLinear(256, 128, max_code=2),
                          DiscreteRatchetLinear(128, 64, max_code=3))
    audit = audit_no_master_weights(model)
    assert audit.violations == ()
    assert audit.ratchet_state_bytes == audit.ratchet_weights + (128 + 64) * 4
    assert compare_persistent_footprint(model).reduction_ratio > 10
    bad = nn.Sequential(DiscreteRatchetLinear(3, 2, max_code=2))
    bad[0].register_parameter("master_weight", nn.Parameter(torch.zeros(2, 3)))
    with pytest.raises(RuntimeError, match="master_weight"):
        audit_no_master_weights(bad, raise_on_violation=True)


def test_trainable_scale_is_one_parameter_per_row():
    layer = DiscreteRatchetLinear(4, 3, max_code=2, trainable_scale=True)
    params = dict(layer.named_parameters())
    assert set(params) == {"log_scale"} and params["log_scale"].shape == (3,)


def tiny_config(**kw) -> ModelConfig:
    return ModelConfig(vocab_size=11, block_size=8, n_layer=2, n_head=2, n_embd=16, **kw)


def test_model_uses_ratchet_layers_everywhere_and_shares_seeded_init():
    # tests/test_model.py:21-38, 90-107
    model = build_seeded_model(tiny_config(), max_code=2, seed=9)
    assert not any(isinstance(m, nn.Linear) for m in model.modules())
    assert audit_no_master_weights(model, raise_on_violation=True).ratchet_layers == 9
    a = build_seeded_model(tiny_config(matmul_mode="bf16"), max_code=3, seed=123)
    b = build_seeded_model(tiny_config(matmul_mode="int8"), max_code=3, seed=123)
    for la, lb in zip([m for m in a.modules() if isinstance(m, DiscreteRatchetLinear)],
                      [m for m in b.modules() if isinstance(m, DiscreteRatchetLinear)]):
        assert torch.equal(la.packed, lb.packed) and torch.equal(la.scale, lb.scale)


def test_model_config_validation():
    with pytest.raises(ValueError, match="matmul_mode"):
        ModelConfig(vocab_size=11, matmul_mode="tf32")
    with pytest.raises(ValueError, match="block_size"):
        RatchetGPT(tiny_config(), max_code=2)(torch.zeros((1, 9), dtype=torch.long))
    assert ModelConfig(vocab_size=8, n_embd=2048, n_head=16, ffn_hidden=5632).hidden_size == 5632
    assert ModelConfig(vocab_size=8, n_embd=64, n_head=4).hidden_size == 256
