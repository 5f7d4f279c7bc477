"""The fused SR-quant + int8 grad_input kernel (rk_grad_input_sr, torch.ops.ratchet.grad_input_sr)
against the two kernels it replaces, bit for bit: the stochastic row quantization of the
gradient (rk_quantize_rows, itself pinned to the oracle's Philox and rounding) followed by
the int8 GEMM on the packed state (rk_int8_gemm_packed_t).

Cases: the op shape's grad_input (16384 x 2048 gradient, 512 outputs), the 25M qkv gradient in
three parts, a float32 gradient quantized as bf16 with the bf16 side output, ragged rows,
one and three contraction steps, 128 / 256 output columns, septenary codes, a device seed
with a row offset, the optional int8 code output, and the argument checks."""

from __future__ import annotations

import pytest
import torch

from helpers import synthetic_state
from local_ai_training import _native as nat
from local_ai_training.int8_matmul import grad_input_sr_supported
from local_ai_training.ops import ratchet

pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


def operands(m, k, n, mc, dtype, nparts, seed, cuda):
    g = gen(seed)
    whole = torch.randn(m, k, generator=g) * 1e-2
    whole[::5, 3] = 0.5      # rows whose absmax sits at different columns
    whole[2::7, -1] = -0.75
    whole = whole.to(dtype).to(cuda)
    parts = [p.contiguous() for p in whole.chunk(nparts, dim=-1)] if nparts > 1 else [whole]
    packed, _ = synthetic_state(k, n, mc, seed=seed + 1)
    cs = (torch.rand(k, generator=g) * 0.02 + 1e-3).to(cuda)
    return whole, parts, torch.from_numpy(packed).to(cuda), cs


CASES = [
    # (M, K, N, max_code, gradient dtype, parts, output dtype, col_scale)
    (16384, 2048, 512, 2, torch.bfloat16, 1, torch.bfloat16, True),   # op shape
    (16384, 1536, 512, 2, torch.bfloat16, 3, torch.bfloat16, True),   # 25M qkv in parts
    (4096, 512, 512, 2, torch.float32, 1, torch.float32, True),       # float32 gradient
    (1000, 192, 128, 3, torch.bfloat16, 1, torch.float32, False),     # ragged rows, 3 steps
    (65, 64, 256, 1, torch.float32, 1, torch.bfloat16, True),         # one step, 65 rows
    (777, 4096, 256, 3, torch.bfloat16, 2, torch.bfloat16, True),     # widest contraction
]


@pytest.mark.parametrize("m,k,n,mc,dtype,nparts,odt,use_cs", CASES)
def test_grad_input_sr_equals_quant_then_gemm(cuda, m, k, n, mc, dtype, nparts, odt, use_cs):
    print(f"grad_input_sr m={m} k={k} n={n} mc={mc} {dtype} parts={nparts} {odt}", flush=True)
    R = ratchet()
    whole, parts, packed, cs = operands(m, k, n, mc, dtype, nparts, 11, cuda)
    cs = cs if use_cs else None
    assert grad_input_sr_supported(parts, packed, cs)
    q_out = torch.full((m, k), 99, dtype=torch.int8, device=cuda)
    out, s = R.grad_input_sr(parts, packed, mc, cs, 4242, None, 0, odt, False, q_out)
    q_ref, s_ref = R.quantize_rows(whole, cs, True, 4242)
    out_ref = R.packed_mm_t(q_ref, packed, mc, s_ref, None, odt)
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref)
    assert torch.equal(q_out, q_ref)
    assert out.dtype == odt and torch.equal(out, out_ref)


def test_grad_input_sr_float32_as_bf16_with_bf16_copy(cuda):
    R = ratchet()
    m, k, n, mc = 2048, 512, 512, 2
    whole, parts, packed, cs = operands(m, k, n, mc, torch.float32, 1, 12, cuda)
    xb = torch.empty(m, k, dtype=torch.bfloat16, device=cuda)
    out, s = R.grad_input_sr(parts, packed, mc, cs, 77, None, 0, torch.float32, True, None, xb)
    xb_ref = torch.empty_like(xb)
    q_ref, s_ref = R.quantize_rows(whole, cs, True, 77, x_bf16=xb_ref, round_bf16=True)
    out_ref = R.packed_mm_t(q_ref, packed, mc, s_ref, None, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(xb, whole.to(torch.bfloat16)) and torch.equal(xb, xb_ref)
    assert torch.equal(s, s_ref) and torch.equal(out, out_ref)


def test_grad_input_sr_device_seed_and_row_offset(cuda):
    R = ratchet()
    m, k, n, mc = 3000, 1024, 512, 2
    whole, parts, packed, cs = operands(m, k, n, mc, torch.bfloat16, 1, 13, cuda)
    slot = torch.tensor([(7 << 40) + 5], dtype=torch.int64, device=cuda)
    out, s = R.grad_input_sr(parts, packed, mc, cs, 0, slot, 12345)
    q_ref, s_ref = R.quantize_rows(whole, cs, True, 0, slot, row_offset=12345)
    out_ref = R.packed_mm_t(q_ref, packed, mc, s_ref, None, torch.bfloat16)
    host, _ = R.grad_input_sr(parts, packed, mc, cs, (7 << 40) + 5, None, 12345)
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref) and torch.equal(out, out_ref) and torch.equal(host, out)


def test_grad_input_sr_through_the_c_abi(cuda):
    m, k, n, mc = 512, 256, 128, 2
    whole, parts, packed, cs = operands(m, k, n, mc, torch.bfloat16, 1, 14, cuda)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=cuda)
    s = torch.empty(m, device=cuda)
    nat.call("rk_grad_input_sr", whole.data_ptr(), None, None, 1, k, nat.RK_BF16, k,
             cs.data_ptr(), 99, None, 0, packed.data_ptr(), n, mc, m, k, n, s.data_ptr(), None,
             k, None, k, out.data_ptr(), nat.RK_BF16, n, nat.stream_handle(cuda))
    q_ref, s_ref = ratchet().quantize_rows(whole, cs, True, 99)
    out_ref = ratchet().packed_mm_t(q_ref, packed, mc, s_ref, None, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref) and torch.equal(out, out_ref)


def test_grad_input_sr_rejects_unsupported_shapes(cuda):
    R = ratchet()
    g = torch.zeros(64, 128, dtype=torch.bfloat16, device=cuda)
    for n in (384, 1024, 136):
        packed = torch.zeros(128, n, dtype=torch.uint8, device=cuda)
        assert not grad_input_sr_supported([g], packed)
        with pytest.raises(RuntimeError, match="fused SR grad_input"):
            R.grad_input_sr([g], packed, 2)
    packed = torch.zeros(96, 128, dtype=torch.uint8, device=cuda)
    with pytest.raises(RuntimeError, match="fused SR grad_input"):
        R.grad_input_sr([g[:, :96]], packed, 2)
    with pytest.raises(RuntimeError, match="packed state"):
        R.grad_input_sr([g], torch.zeros(64, 128, dtype=torch.uint8, device=cuda), 2)
    with pytest.raises(RuntimeError, match="round_bf16"):
        R.grad_input_sr([g], torch.zeros(128, 128, dtype=torch.uint8, device=cuda), 2,
                        round_bf16=True)
