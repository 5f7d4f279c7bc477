"""Gradients read in parts: the SR row quantization and the bf16 grad_weight partials of a
gradient given as up to three [M, C] pieces of one row (torch.ops.ratchet.quantize_rows_parts,
grad_weight_partials_parts and their C-ABI entry points) against the same kernels on the
concatenated rows, bit for bit.

The qkv layer's backward receives dq, dk and dv as three separate allocations; quantizing
and multiplying them in place must give exactly the codes, scales and partials of the
concatenation torch.cat(dq, dk, dv) that it replaces (int8_matmul.py:142 rounding, the same
Philox draw per (row, column) of the whole row)."""

from __future__ import annotations

import pytest
import torch

from local_ai_training import _native as nat
from local_ai_training.int8_matmul import grad_weight_parts_supported
from local_ai_training.ops import ratchet

pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


def pieces(m, c, n, dtype, seed, cuda, layout):
    g = gen(seed)
    whole = (torch.randn(m, n * c, generator=g) * 1e-2).to(dtype)
    # a few rows with a large value, so the row absmax comes from different parts
    whole[::7, -1] = 3.0
    whole[1::7, 0] = -2.5
    whole = whole.to(cuda)
    if layout == "views":
        return whole, list(whole.chunk(n, dim=-1))
    parts = [p.contiguous() for p in whole.chunk(n, dim=-1)]
    return torch.cat(parts, dim=-1), parts


CASES = [
    # (M, C, parts, dtype, layout)
    (16384, 512, 3, torch.bfloat16, "separate"),  # 25M qkv gradient shape
    (333, 256, 3, torch.float32, "separate"),     # ragged rows, float32 gradient
    (96, 128, 2, torch.bfloat16, "views"),        # chunks of one [M, 2C] tensor
    (64, 72, 3, torch.bfloat16, "separate"),      # part width not a multiple of 64
    (40, 256, 1, torch.bfloat16, "separate"),
]


@pytest.mark.parametrize("m,c,n,dtype,layout", CASES)
@pytest.mark.parametrize("stochastic", [False, True])
def test_quantize_rows_parts_equals_quantizing_the_concatenation(cuda, m, c, n, dtype, layout,
                                                                  stochastic):
    print(f"quantize parts m={m} c={c} n={n} {dtype} {layout} sr={stochastic}", flush=True)
    R = ratchet()
    whole, parts = pieces(m, c, n, dtype, 1, cuda, layout)
    col_scale = (torch.rand(n * c, generator=gen(2)) + 0.5).to(cuda)
    for cs in (None, col_scale):
        q, s = R.quantize_rows_parts(parts, cs, stochastic, 9876)
        q_ref, s_ref = R.quantize_rows(whole, cs, stochastic, 9876)
        torch.cuda.synchronize()
        assert torch.equal(q, q_ref) and torch.equal(s, s_ref)


def test_quantize_rows_parts_with_a_device_seed_and_row_offset(cuda):
    R = ratchet()
    whole, parts = pieces(512, 256, 3, torch.bfloat16, 3, cuda, "separate")
    slot = torch.tensor([2 ** 40 + 17], dtype=torch.int64, device=cuda)
    q, s = R.quantize_rows_parts(parts, None, True, 0, slot, 4096)
    q_ref, s_ref = R.quantize_rows(whole, None, True, 0, slot, row_offset=4096)
    # the host seed of the same value gives the same draw
    q_host, _ = R.quantize_rows_parts(parts, None, True, 2 ** 40 + 17, None, 4096)
    torch.cuda.synchronize()
    assert torch.equal(q, q_ref) and torch.equal(s, s_ref) and torch.equal(q, q_host)


GW_CASES = [
    # (M, C, parts, K, layout)
    (16384, 512, 3, 512, "separate"),  # 25M qkv: [1536, 512] weight gradient
    (2048, 2048, 3, 2048, "separate"),  # 1B qkv width (large output tiles), fewer rows
    (300, 256, 2, 128, "views"),
    (96, 128, 3, 160, "separate"),
]


@pytest.mark.parametrize("m,c,n,k,layout", GW_CASES)
def test_grad_weight_partials_parts_equal_those_of_the_concatenation(cuda, m, c, n, k, layout):
    print(f"grad_weight parts m={m} c={c} n={n} k={k} {layout}", flush=True)
    R = ratchet()
    whole, parts = pieces(m, c, n, torch.bfloat16, 4, cuda, layout)
    g = gen(5)
    q = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(cuda)
    s = (torch.rand(m, generator=g) * 0.05 + 1e-3).to(cuda)
    assert grad_weight_parts_supported(parts, q)
    nsplit = R.grad_weight_splits(m, n * c, k)
    work = torch.full((nsplit, n * c, k), float("nan"), device=cuda)
    work_ref = torch.full_like(work, float("nan"))
    R.grad_weight_partials_parts(parts, q, s, work)
    R.grad_weight_partials(whole, q, s, work_ref)
    # the dequantized bf16 activations give the same partials
    xd = R.dequant_bf16(q, s)
    work_x = torch.full_like(work, float("nan"))
    R.grad_weight_partials_parts(parts, xd, None, work_x)
    torch.cuda.synchronize()
    assert torch.equal(work, work_ref) and torch.equal(work_x, work_ref)


def test_parts_through_the_c_abi(cuda):
    m, c, k = 256, 256, 128
    whole, parts = pieces(m, c, 3, torch.bfloat16, 6, cuda, "separate")
    stream = nat.stream_handle(cuda)
    q = torch.empty(m, 3 * c, dtype=torch.int8, device=cuda)
    s = torch.empty(m, device=cuda)
    p = [t.data_ptr() for t in parts]
    nat.call("rk_quantize_rows_parts", *p, 3, c, nat.RK_BF16, m, c, None, 1, 31337, None, 0,
             q.data_ptr(), 3 * c, s.data_ptr(), stream)
    q_ref, s_ref = ratchet().quantize_rows(whole, None, True, 31337)
    g = gen(7)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(cuda)
    sa = (torch.rand(m, generator=g) * 0.05 + 1e-3).to(cuda)
    out = torch.empty(3 * c, k, dtype=torch.bfloat16, device=cuda)
    nsplit = ratchet().grad_weight_splits(m, 3 * c, k)
    work = torch.empty(nsplit, 3 * c, k, device=cuda)
    nat.call("rk_grad_weight_bf16_parts", *p, 3, c, nat.RK_BF16, c, a.data_ptr(), nat.RK_I8, k,
             sa.data_ptr(), m, 3 * c, k, work.data_ptr(), nsplit, out.data_ptr(), k, stream)
    torch.cuda.synchronize()
    assert torch.equal(q, q_ref) and torch.equal(s, s_ref)
    assert torch.equal(out, ratchet().grad_weight(whole, a, sa))


def test_parts_reject_bad_arguments(cuda):
    R = ratchet()
    parts = [torch.zeros(8, 128, dtype=torch.bfloat16, device=cuda) for _ in range(3)]
    q = torch.zeros(8, 128, dtype=torch.int8, device=cuda)
    s = torch.ones(8, device=cuda)
    with pytest.raises(RuntimeError, match="1 to 3 parts"):
        R.quantize_rows_parts(parts + parts[:1])
    with pytest.raises(RuntimeError, match="share shape"):
        R.quantize_rows_parts([parts[0], torch.zeros(8, 64, dtype=torch.bfloat16, device=cuda)])
    with pytest.raises(RuntimeError, match="share shape"):
        R.quantize_rows_parts([parts[0], parts[1].float()])
    with pytest.raises(RuntimeError, match="unit column stride"):
        R.quantize_rows_parts([parts[0].t()])
    odd = [torch.zeros(8, 96, dtype=torch.bfloat16, device=cuda) for _ in range(3)]
    work = torch.zeros(R.grad_weight_splits(8, 288, 128), 288, 128, device=cuda)
    assert not grad_weight_parts_supported(odd, q)
    with pytest.raises(RuntimeError):
        R.grad_weight_partials_parts(odd, q, s, work)
    with pytest.raises(RuntimeError, match="row scale"):
        R.grad_weight_partials_parts(parts, q, None, work)
    stream = nat.stream_handle(cuda)
    out = torch.empty(8, 384, dtype=torch.int8, device=cuda)
    with pytest.raises(nat.NativeError):
        nat.call("rk_quantize_rows_parts", parts[0].data_ptr(), None, None, 4, 128,
                 nat.RK_BF16, 8, 128, None, 0, 0, None, 0, out.data_ptr(), 384,
                 s.data_ptr(), stream)
