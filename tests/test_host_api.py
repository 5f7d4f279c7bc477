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


def test_captured_step_refuses_sort_based_embedding_backward():
    """The captured training step is refused, before any step runs, wherever the token
    embedding's weight gradient would come from torch's sort-based embedding backward (the
    backward whose memset node a replayed graph must not hold); the HIP path is accepted."""
    from local_ai_training.training import CapturedTrainingStep

    def model(**kw):
        m = RatchetGPT(tiny_config(**kw), max_code=2)
        return m

    plain = model()
    assert not plain.embedding_backward_is_sort_based()
    off = model()
    off.hip_embedding_backward = False
    assert off.embedding_backward_is_sort_based()
    ratchet_emb = model(ratchet_embedding=True)
    assert ratchet_emb.embedding_backward_is_sort_based()
    padded = model()
    padded.token_embedding.padding_idx = 0
    assert padded.embedding_backward_is_sort_based()
    for attr, value in (("max_norm", 1.0), ("sparse", True), ("scale_grad_by_freq", True)):
        m = model()
        setattr(m.token_embedding, attr, value)
        assert m.embedding_backward_is_sort_based(), attr
    wide = RatchetGPT(ModelConfig(vocab_size=11, block_size=8, n_layer=1, n_head=2,
                                  n_embd=4098), max_code=2)
    assert wide.embedding_backward_is_sort_based()
    frozen = model()
    frozen.token_embedding.weight.requires_grad_(False)
    frozen.hip_embedding_backward = False
    assert not frozen.embedding_backward_is_sort_based()

    tokens = torch.zeros((1, 8), dtype=torch.long)
    for bad in (off, ratchet_emb, padded):
        opt = torch.optim.AdamW([p for p in bad.parameters() if p.requires_grad], lr=1e-3)
        with pytest.raises(RuntimeError, match="sort-based embedding backward"):
            CapturedTrainingStep(bad, opt, tokens, tokens)


def test_attention_gate_repeats_the_kernel_extent_check():
    """attention_supported sends inputs whose per-head extent would overflow the kernel's
    32-bit offsets to torch's attention instead of letting the HIP op raise (the gate alone,
    on shapes and strides; no allocation)."""
    from local_ai_training.attention import _extent_fits

    # the 25M and 1B shapes as the model's strided views ([B, S, 3, H, D] -> [B, H, S, D])
    assert _extent_fits((32, 8, 512, 64), (512 * 3 * 512, 64, 3 * 512, 1))
    assert _extent_fits((8, 16, 1024, 128), (1024 * 3 * 2048, 128, 3 * 2048, 1))
    # a row stride whose (S + 128) rows pass 2^31 bytes, just under and just over
    d = 128
    s = 4096
    limit = (2**31 // 2 - d) // (s + 128)
    assert _extent_fits((1, 1, s, d), (0, 0, limit, 1))
    assert not _extent_fits((1, 1, s, d), (0, 0, limit + 1, 1))
    assert not _extent_fits((2**16, 2**15 + 1, 1, 64), (0, 0, 64, 1))
