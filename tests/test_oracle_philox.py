"""Pins the oracle's Philox4x32-10 and the [0, 1) map used for stochastic rounding."""

import numpy as np

from oracle import philox


def _h(s: str) -> int:
    return int(s, 16)


def test_philox_matches_random123_known_answers(golden):
    for vec in golden["philox4x32_10"]["vectors"]:
        ctr = [np.array([_h(c)], dtype=np.uint32) for c in vec["ctr"]]
        k0, k1 = (_h(k) for k in vec["key"])
        out = philox.philox4x32(*ctr, k0, k1, rounds=10)
        assert [f"{int(o[0]):08x}" for o in out] == vec["out"]


def test_randint_uses_offset_as_first_counter_word_and_seed_as_key():
    # counter (offset, 0, 0, 0), key (seed lo, seed hi): the first Random123 vector is
    # offset 0 / seed 0.
    assert int(philox.randint(0, [0])[0]) == 0x6627E8D5
    seed = 0x299F31D0_A4093822
    full = philox.philox4x32(np.array([7], np.uint32), 0, 0, 0, 0xA4093822, 0x299F31D0)
    assert int(philox.randint(seed, [7])[0]) == int(full[0][0])


def test_uniform_map_closed_form_endpoints():
    words = np.array([0x00000000, 0x00000001, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF, 0xFFFFFFFE],
                     dtype=np.uint32)
    u = philox.uint_to_uniform_float(words)
    scale = np.float32(2.0**-31 - 2.0**-55)  # float32 0x2FFFFFFF
    assert philox.UNIFORM_SCALE.view(np.uint32) == 0x2FFFFFFF
    assert u[0] == 0.0
    assert u[1] == scale
    # 2**31 - 1 rounds to 2**31 in float32; times the scale gives 1 - 2**-24 (< 1).
    assert u[2] == np.float32(1.0 - 2.0**-24)
    assert u[3] == u[2]  # INT_MIN maps to INT_MAX
    assert u[4] == 0.0  # -1 maps to 0
    assert u[5] == scale  # -2 maps to 1


def test_uniform_values_lie_in_unit_interval_and_are_roughly_uniform():
    u = philox.rand(12345, np.arange(200_000, dtype=np.uint32))
    assert u.dtype == np.float32
    assert float(u.min()) >= 0.0 and float(u.max()) < 1.0
    hist, _ = np.histogram(u, bins=10, range=(0.0, 1.0))
    assert np.all(np.abs(hist - 20_000) < 1_000)


def test_sr_offsets_wrap_like_int32_products():
    rows, cols = 3, 70_001
    off = philox.sr_offsets(rows, cols, row_start=70_000)
    for m, k in ((0, 0), (1, 12), (2, 70_000)):
        assert int(off[m, k]) == ((70_000 + m) * cols + k) % 2**32
