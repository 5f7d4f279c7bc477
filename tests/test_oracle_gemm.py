"""Pins the oracle's scaled int8 GEMM and bf16 rounding."""

import numpy as np
import torch

from oracle import gemm
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits


def test_int_matmul_matches_brute_force():
    rng = np.random.default_rng(0)
    a = rng.integers(-127, 128, size=(3, 5), dtype=np.int8)
    b = rng.integers(-7, 8, size=(5, 4), dtype=np.int8)
    expected = [[sum(int(a[i, k]) * int(b[k, j]) for k in range(5)) for j in range(4)]
                for i in range(3)]
    assert gemm.int_matmul(a, b).tolist() == expected


def test_scaled_mm_matches_reference_formula_for_non_tile_shape():
    # tests/test_int8_matmul.py:172-187, evaluated with torch on the CPU.
    g = torch.Generator().manual_seed(3)
    lhs = torch.randint(-20, 21, (67, 35), generator=g, dtype=torch.int8)
    rhs = torch.randint(-8, 9, (35, 53), generator=g, dtype=torch.int8)
    ls = torch.rand(67, generator=g) + 0.01
    rs = torch.rand(53, generator=g) + 0.01
    expected = ((lhs.float() @ rhs.float()) * ls[:, None] * rs[None, :]).to(torch.bfloat16)
    got = gemm.scaled_int8_mm(lhs.numpy(), rhs.numpy(), ls.numpy(), rs.numpy())
    assert np.array_equal(got, expected.view(torch.int16).numpy().view(np.uint16))


def test_epilogue_without_rhs_scale_is_row_scale_only():
    acc = np.array([[3, -5], [7, 0]], dtype=np.int64)
    ls = np.array([0.5, 2.0], np.float32)
    out = gemm.scaled_epilogue(acc, ls, None)
    assert out.tolist() == [[1.5, -2.5], [14.0, 0.0]]


def test_bf16_rounding_matches_torch_including_specials():
    g = torch.Generator().manual_seed(5)
    vals = torch.cat([
        torch.randn(10_000, generator=g) * 1e3,
        torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 1e-40, -3e-39,
                      3.3895314e38, 1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8]),
    ])
    ours = f32_to_bf16_bits(vals.numpy())
    theirs = vals.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    # NaN payloads differ between torch's CPU conversion paths; only NaN-ness matters.
    nan = np.isnan(vals.numpy())
    assert np.array_equal(ours[~nan], theirs[~nan])
    assert np.all(np.isnan(bf16_bits_to_f32(ours[nan])))
    assert np.array_equal(bf16_bits_to_f32(ours), vals.to(torch.bfloat16).float().numpy(),
                          equal_nan=True)
