"""The dequantized activations written by the activation quantizations (the ``_dq`` entry
points: rk_quantize_rows_dq, rk_rmsnorm_quantize_dq, rk_gelu_quantize_dq,
rk_transpose_quantize_dq, and the ``x_dq`` argument of their operators).

Each must give the same int8 rows and scales as the call without the output, and
x_dq = bf16(bf16(q) * bf16(s)) bit for bit: the dequantized copy ratchet.py:73-75 forms for the
bf16 grad_weight, as rk_dequant_bf16 computes it (itself checked against the oracle's
dequantization), so the backward reading x_dq sees exactly the operand it would convert from
q and s."""

from __future__ import annotations

import pytest
import torch

from local_ai_training import _native as nat
from local_ai_training.ops import ratchet

pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


SHAPES = [(4096, 512), (333, 2048), (77, 136), (5, 8)]  # ragged: 136 % 64 != 0, tiny rows


@pytest.mark.parametrize("m,k", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quantizations_write_the_dequantized_rows(cuda, m, k, dtype):
    print(f"dequant m={m} k={k} {dtype}", flush=True)
    R = ratchet()
    x = (torch.randn(m, k, generator=gen(1)) * 2).to(dtype).to(cuda)
    w = (torch.rand(k, generator=gen(2)) + 0.5).to(cuda)
    cases = [
        ("plain", lambda dq: R.quantize_rows(x, x_dq=dq), lambda: R.quantize_rows(x)),
        ("rmsnorm", lambda dq: R.rmsnorm_quantize(x, w, 1e-5, dq),
         lambda: R.rmsnorm_quantize(x, w, 1e-5)),
        ("gelu", lambda dq: R.gelu_quantize(x, dq), lambda: R.gelu_quantize(x)),
    ]
    if k % 4 == 0:
        att = x.view(1, m, 4, k // 4).transpose(1, 2)  # [B, H, S, D], strided
        cases.append(("transpose", lambda dq: R.transpose_quantize(att, dq),
                      lambda: R.transpose_quantize(att)))
    for name, with_dq, plain in cases:
        dq = torch.full((m, k), float("nan"), dtype=torch.bfloat16, device=cuda)
        q, s = with_dq(dq)
        q_ref, s_ref = plain()
        torch.cuda.synchronize()
        assert torch.equal(q, q_ref) and torch.equal(s, s_ref), name
        assert torch.equal(dq, R.dequant_bf16(q, s)), name


def test_dequantized_rows_through_the_c_abi(cuda):
    m, k = 256, 512
    x = torch.randn(m, k, generator=gen(3)).to(cuda)
    q = torch.empty(m, k, dtype=torch.int8, device=cuda)
    s = torch.empty(m, device=cuda)
    dq = torch.empty(m, k + 8, dtype=torch.bfloat16, device=cuda)  # padded rows
    stream = nat.stream_handle(cuda)
    nat.call("rk_quantize_rows_dq", x.data_ptr(), nat.RK_F32, m, k, k, 1, q.data_ptr(), k,
             s.data_ptr(), dq.data_ptr(), k + 8, stream)
    w = torch.ones(k, device=cuda)
    q2, s2 = torch.empty_like(q), torch.empty_like(s)
    dq2 = torch.empty(m, k, dtype=torch.bfloat16, device=cuda)
    nat.call("rk_rmsnorm_quantize_dq", x.data_ptr(), nat.RK_F32, k, w.data_ptr(), 1e-5,
             q2.data_ptr(), k, s2.data_ptr(), m, k, dq2.data_ptr(), k, stream)
    torch.cuda.synchronize()
    R = ratchet()
    assert torch.equal(dq[:, :k], R.dequant_bf16(q, s))
    assert torch.equal(dq2, R.dequant_bf16(q2, s2))
    with pytest.raises(nat.NativeError, match="x_dq"):
        nat.call("rk_gelu_quantize_dq", x.data_ptr(), nat.RK_F32, k, q.data_ptr(), k,
                 s.data_ptr(), m, k, dq.data_ptr(), k + 4, stream)  # stride not a multiple of 8


def test_dequantized_output_argument_checks(cuda):
    R = ratchet()
    x = torch.randn(8, 64, device=cuda)
    with pytest.raises(RuntimeError, match="x_dq must be"):
        R.quantize_rows(x, x_dq=torch.empty(8, 64, device=cuda))  # float32
    with pytest.raises(RuntimeError, match="plain round-to-nearest"):
        R.quantize_rows(x, None, True, 5, x_dq=torch.empty(8, 64, dtype=torch.bfloat16,
                                                           device=cuda))
