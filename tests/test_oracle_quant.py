"""Pins the oracle's row quantizers against the reference's torch formula.

The reference's own oracle for the fused quantizers is the tensor expression of
``int8_matmul.py:225-239`` (``_quantize_rows_reference``); the torch CPU evaluation
below is an independent implementation of it, so bit-equality here pins the numpy
oracle (round-half-even, IEEE division, FLT_MIN floor, col pre-scale).
"""

import numpy as np
import pytest
import torch

from oracle import quant
from oracle.numerics import TINY


def torch_quantize_rows(values: torch.Tensor, col_scale: torch.Tensor | None = None):
    prepared = values.float()
    if col_scale is not None:
        prepared = prepared * col_scale.float()[None, :]
    scale = (prepared.abs().amax(dim=1) / 127.0).clamp_min(torch.finfo(torch.float32).tiny)
    q = torch.clamp((prepared / scale[:, None]).round(), -127, 127)
    return q.to(torch.int8), scale


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(67, 35), (128, 256), (1, 513), (255, 1), (300, 2048)])
def test_row_quant_matches_torch_formula(shape, dtype):
    g = torch.Generator().manual_seed(7)
    values = (torch.randn(shape, generator=g) * 3.0).to(dtype)
    q_ref, s_ref = torch_quantize_rows(values)
    q, s = quant.quantize_rows(values.float().numpy())
    assert np.array_equal(q, q_ref.numpy())
    assert np.array_equal(s.view(np.uint32), s_ref.numpy().view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_colscaled_quant_matches_torch_formula(dtype):
    g = torch.Generator().manual_seed(21)
    values = (torch.randn(67, 35, generator=g) * 3.0).to(dtype)
    col = torch.rand(35, generator=g) + 0.01
    q_ref, s_ref = torch_quantize_rows(values, col)
    q, s = quant.quantize_rows(values.float().numpy(), col.numpy())
    assert np.array_equal(q, q_ref.numpy())
    assert np.array_equal(s, s_ref.numpy())


def test_noncontiguous_view_matches():
    g = torch.Generator().manual_seed(11)
    base = (torch.randn(70, 48, generator=g) * 2.0).to(torch.bfloat16)
    view = base.t()
    q_ref, s_ref = torch_quantize_rows(view)
    q, s = quant.quantize_rows(view.float().numpy())
    assert np.array_equal(q, q_ref.numpy()) and np.array_equal(s, s_ref.numpy())


def test_ties_round_half_to_even():
    # amax 127 -> scale exactly 1.0; the .5 cases must round to even.
    row = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -2.5, 3.5, -126.5]], dtype=np.float32)
    q, s = quant.quantize_rows(row)
    assert s[0] == 1.0
    assert q.tolist() == [[127, 0, 2, 2, 0, -2, 4, -126]]


def test_zero_rows_give_tiny_scale_and_zero_codes():
    q, s = quant.quantize_rows(np.zeros((3, 5), np.float32))
    assert np.count_nonzero(q) == 0
    assert np.all(s == TINY) and np.all(np.isfinite(s))


def test_stochastic_rounding_brackets_and_is_unbiased():
    rng = np.random.default_rng(31)
    x = rng.standard_normal((8, 64)).astype(np.float32)
    col = np.ones(64, np.float32)
    q_det, scale = quant.quantize_rows(x, col)
    y = x / scale[:, None]
    acc = np.zeros_like(x, dtype=np.float64)
    draws = 400
    for seed in range(draws):
        q, s = quant.quantize_rows_sr(x, col, seed)
        assert np.array_equal(s, scale)
        assert np.all((q == np.floor(y)) | (q == np.floor(y) + 1) | (np.abs(q) == 127))
        acc += q.astype(np.float64) * s[:, None]
    mean = acc / draws
    rel = np.abs(mean - x).mean() / scale.mean()
    assert rel < 0.1
    # a deterministic rounding would be biased per element; SR's empirical mean is not.
    assert np.abs(mean - x).mean() < np.abs(q_det * scale[:, None] - x).mean()


def test_stochastic_rounding_rate_equals_fractional_part():
    # y = 0.25 quant steps: P(round up) must be 0.25 (floor(y + u), u ~ U[0,1)).
    x = np.zeros((1, 4096), np.float32)
    x[0, 0] = 127.0  # scale = 1
    x[0, 1:] = 0.25
    q, _ = quant.quantize_rows_sr(x, None, seed=99)
    rate = q[0, 1:].mean()
    assert abs(rate - 0.25) < 0.03


def test_stochastic_rounding_is_seed_deterministic():
    x = np.random.default_rng(0).standard_normal((5, 33)).astype(np.float32)
    a, _ = quant.quantize_rows_sr(x, None, 7)
    b, _ = quant.quantize_rows_sr(x, None, 7)
    c, _ = quant.quantize_rows_sr(x, None, 8)
    assert np.array_equal(a, b) and not np.array_equal(a, c)


def test_column_quant_is_row_quant_of_transpose():
    x = np.random.default_rng(1).standard_normal((40, 9)).astype(np.float32)
    q, s = quant.quantize_columns(x)
    qt, st = quant.quantize_rows(x.T)
    assert np.array_equal(q, qt.T) and np.array_equal(s, st)
