"""The embedding-gradient oracle against torch's own embedding backward on the CPU (the
reference model's op, model.py:219/237): bit-exact on integer-valued gradients, where every
summation order gives the same float32 sums, and within reassociation error on floats."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.embedding import CHUNK, embedding_backward


def torch_grad(g: np.ndarray, ids: np.ndarray, v: int) -> np.ndarray:
    w = torch.zeros(v, g.shape[1], requires_grad=True)
    torch.nn.functional.embedding(torch.from_numpy(ids), w).backward(torch.from_numpy(g))
    return w.grad.numpy()


@pytest.mark.parametrize("t,v,d", [(0, 5, 4), (1, 3, 8), (63, 7, 4), (64, 64, 12),
                                   (1000, 50, 20), (5000, 9, 16)])
def test_integer_gradients_bit_exact_with_torch(t, v, d):
    rng = np.random.default_rng(t + v + d)
    ids = rng.integers(0, v, t)
    g = rng.integers(-64, 65, (t, d)).astype(np.float32)
    assert np.array_equal(embedding_backward(g, ids, v), torch_grad(g, ids, v))


def test_float_gradients_close_to_torch_and_unused_rows_zero():
    rng = np.random.default_rng(7)
    ids = np.minimum(rng.zipf(1.1, 4000) - 1, 299)
    g = rng.standard_normal((4000, 32)).astype(np.float32) * 1e-3
    got = embedding_backward(g, ids, 400)
    # reassociation only (the worst-case bound (n - 1) * 2^-24 * sum |g| is far looser)
    np.testing.assert_allclose(got, torch_grad(g, ids, 400), rtol=1e-5, atol=1e-7)
    assert not got[300:].any()


def test_fixed_order_is_chunked_then_chunk_order():
    # three rows of one id: 1, then 2^-24 twice. In one chunk the sum is sequential:
    # (1 + 2^-24) + 2^-24 = 1 (each add rounds to even). With the first row in an earlier
    # chunk, the later chunk first sums 2^-24 + 2^-24 = 2^-23 exactly and 1 + 2^-23 is exact.
    tiny = np.float32(2.0 ** -24)
    g = np.zeros((CHUNK + 2, 1), dtype=np.float32)
    g[0, 0], g[CHUNK, 0], g[CHUNK + 1, 0] = 1.0, tiny, tiny
    ids = np.full(CHUNK + 2, 1)
    ids[0] = 0
    ids[CHUNK - 1] = 0
    ids[CHUNK:] = 0
    ids[1:CHUNK - 1] = 1
    got = embedding_backward(g, ids, 2)
    assert got[0, 0] == np.float32(1.0) + np.float32(2.0 ** -23)
    same_chunk = embedding_backward(g, ids, 2, chunk=2 * CHUNK)
    assert same_chunk[0, 0] == np.float32(1.0)


def test_ids_outside_the_table_are_dropped():
    g = np.ones((5, 4), dtype=np.float32)
    got = embedding_backward(g, np.array([0, 3, -1, 7, 3]), 4)
    assert got[0, 0] == 1 and got[3, 0] == 2 and got[1:3].sum() == 0
