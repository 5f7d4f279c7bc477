"""Pins the oracle's integer ratchet update and row normalization.

Known answers come from the reference's own tests (tests/test_ratchet.py) and are
read from tests/golden/reference_vectors.json.
"""

import numpy as np
import pytest
import torch

from helpers import reference_init
from oracle import update


def test_bucket_pressure_known_answer(golden):
    kat = golden["bucket_pressure"]
    z = np.array(kat["z"], np.float32)
    assert update.bucket_pressure(z, kat["low"], kat["high"]).tolist() == kat["expected"]


def test_positive_gradient_click_known_answer(golden):
    kat = golden["positive_click"]
    mc, T = kat["max_code"], kat["threshold"]
    code, _ = reference_init(1, 2, mc, torch.tensor(kat["reference_weight"]))
    packed = update.pack(code, np.zeros_like(code), mc)
    new, counts = update.update_core(packed, np.array(kat["z"], np.float32), mc, T)
    c, p = update.unpack(new, mc)
    assert c.tolist() == kat["code_after"] and p.tolist() == kat["pressure_after"]
    assert counts[1] == kat["negative_moves"] and counts[0] == kat["positive_moves"]


def test_saturated_click_known_answer(golden):
    kat = golden["saturated_click"]
    mc, T = kat["max_code"], kat["threshold"]
    code = np.array(kat["code_before"], np.int8)
    packed = update.pack(code, np.zeros_like(code), mc)
    new, counts = update.update_core(packed, np.array(kat["z"], np.float32), mc, T)
    c, p = update.unpack(new, mc)
    assert c.tolist() == kat["code_after"] and p.tolist() == kat["pressure_after"]
    assert counts[2] == kat["blocked_positive_moves"] and counts[0] == kat["positive_moves"]


@pytest.mark.parametrize("max_code", [1, 2, 3, 4, 5, 6, 7])
def test_pack_unpack_round_trip(max_code):
    codes = np.arange(-max_code, max_code + 1, dtype=np.int8)
    pressures = np.arange(-7, 8, dtype=np.int8)
    cg, pg = np.meshgrid(codes, pressures, indexing="ij")
    packed = update.pack(cg, pg, max_code)
    c, p = update.unpack(packed, max_code)
    assert np.array_equal(c, cg) and np.array_equal(p, pg)


def test_golden_sixty_step_update(golden):
    kat = golden["golden_60_step_update"]
    for case in kat["cases"]:
        mc = case["max_code"]
        torch.manual_seed(kat["seed"])
        code, _ = reference_init(kat["out_features"], kat["in_features"], mc)
        packed = update.pack(code, np.zeros_like(code), mc)
        total = 0
        for _ in range(kat["steps"]):
            z = (torch.randn(kat["out_features"], kat["in_features"])
                 * kat["gradient_scale"]).numpy()
            packed, counts = update.update_core(packed, z, mc, kat["threshold"])
            total += int(counts[0] + counts[1])
        c, p = update.unpack(packed, mc)
        assert int(c.astype(np.int64).sum()) == case["code_sum"]
        assert int(p.astype(np.int64).sum()) == case["pressure_sum"]
        assert total == case["total_moves"]


def test_stored_pressure_stays_within_nibble_under_adversarial_updates():
    # tests/test_ratchet.py:224-233
    torch.manual_seed(0)
    for mc in (2, 3, 4):
        for T in (1, 2, 4, 8):
            code, _ = reference_init(6, 8, mc)
            packed = update.pack(code, np.zeros_like(code), mc)
            for step in range(200):
                sign = 1.0 if step % 7 < 5 else -1.0
                z = (sign * (3.0 + torch.rand(6, 8))).numpy()
                packed, _ = update.update_core(packed, z, mc, T)
                c, p = update.unpack(packed, mc)
                assert int(np.abs(p).max()) <= 7 and int(np.abs(c).max()) <= mc


def test_threshold_above_eight_wraps_the_nibble():
    # pressure -8 stored with threshold 9 wraps to +8 in the nibble (ratchet.py:190-192):
    # a documented quirk of the packing, reproduced rather than fixed.
    packed = update.pack(np.array([[0]], np.int8), np.array([[-7]], np.int8), 2)
    new, counts = update.update_core(packed, np.array([[0.6]], np.float32), 2, 9)
    _, p = update.unpack(new, 2)
    assert p.tolist() == [[8]] and counts.sum() == 0


@pytest.mark.parametrize("vec", [4, 8])
@pytest.mark.parametrize("k", [1, 7, 64, 255, 256, 512, 1000, 2048, 5632])
def test_lane_order_sum_counts_every_term_once(vec, k):
    # Small integers: every partial sum is exact, so any order gives the exact total;
    # a dropped, duplicated or misplaced term changes it.
    rng = np.random.default_rng(k * vec)
    g = rng.integers(-8, 9, size=(5, k)).astype(np.float32)
    expected = (g.astype(np.int64) ** 2).sum(axis=1)
    assert np.array_equal(update.row_sumsq(g, vec).astype(np.int64), expected)
    terms = rng.integers(-50, 51, size=(5, k)).astype(np.float32)
    assert np.array_equal(update.lane_order_sum(terms, vec).astype(np.int64),
                          terms.astype(np.int64).sum(axis=1))


def test_normalize_matches_float64_formula():
    rng = np.random.default_rng(3)
    g = (rng.standard_normal((64, 512)) * 1e-3).astype(np.float32)
    z, rms, _ = update.normalize_rows(g, 1e-8, 8)
    ref_rms = np.sqrt((g.astype(np.float64) ** 2).mean(axis=1))
    assert np.allclose(rms, ref_rms, rtol=2e-6)
    ref_z = g / (ref_rms[:, None] + 1e-8)
    assert np.allclose(z, ref_z, rtol=4e-6, atol=0)


def test_rms_ema_first_step_instantaneous_then_smooths():
    # tests/test_ratchet.py:459-472
    rng = np.random.default_rng(0)
    g1 = rng.standard_normal((6, 8)).astype(np.float32)
    ema0 = np.zeros(6, np.float32)
    z1, _, ema1 = update.normalize_rows(g1, 1e-8, 4, ema0, 0.9)
    z_inst, _, _ = update.normalize_rows(g1, 1e-8, 4)
    assert np.array_equal(z1, z_inst)
    g2 = (rng.standard_normal((6, 8)) * 5.0).astype(np.float32)
    z2, _, ema2 = update.normalize_rows(g2, 1e-8, 4, ema1, 0.9)
    ms1 = (g1.astype(np.float64) ** 2).mean(axis=1)
    ms2 = (g2.astype(np.float64) ** 2).mean(axis=1)
    expected = g2 / (np.sqrt(0.9 * ms1 + 0.1 * ms2)[:, None] + 1e-8)
    assert np.allclose(z2, expected, rtol=1e-5)


def test_rms_ema_keeps_value_for_rows_without_gradient():
    g = np.zeros((2, 8), np.float32)
    g[0] = 1.0
    ema = np.array([0.0, 0.5], np.float32)
    _, _, new = update.normalize_rows(g, 1e-8, 4, ema, 0.9)
    assert new[0] == 1.0 and new[1] == np.float32(0.5)


def test_zero_gradient_moves_nothing():
    # tests/test_ratchet.py:109-116
    packed = update.pack(np.zeros((2, 4), np.int8), np.zeros((2, 4), np.int8), 3)
    out = update.update_from_gradient(packed, np.zeros((2, 4), np.float32), 3, 8, 0.5, 1.5,
                                      1e-8, 4)
    assert out["counts"].sum() == 0 and np.array_equal(out["packed"], packed)
    assert np.all(np.isfinite(out["row_rms"]))


def test_nonfinite_rows_are_left_unchanged_and_flagged():
    rng = np.random.default_rng(4)
    code = rng.integers(-2, 3, size=(3, 16)).astype(np.int8)
    packed = update.pack(code, rng.integers(-7, 8, size=(3, 16)).astype(np.int8), 2)
    g = (rng.standard_normal((3, 16)) * 3).astype(np.float32)
    g[1, 5] = np.nan
    out = update.update_from_gradient(packed, g, 2, 2, 0.5, 1.5, 1e-8, 4)
    assert out["nonfinite"] == 1
    assert np.array_equal(out["packed"][1], packed[1])
    clean = update.update_from_gradient(packed[[0, 2]], g[[0, 2]], 2, 2, 0.5, 1.5, 1e-8, 4)
    assert np.array_equal(out["packed"][[0, 2]], clean["packed"])
    assert np.array_equal(out["counts"], clean["counts"])


def test_pressure_leak_moves_toward_zero():
    # tests/test_ratchet.py:489-513
    code = np.zeros((4, 8), np.int8)
    for start, expected in ((5, 4), (-2, -1), (0, 0)):
        packed = update.pack(code, np.full((4, 8), start, np.int8), 2)
        _, p = update.unpack(update.pressure_leak(packed, 2), 2)
        assert np.all(p == expected)
