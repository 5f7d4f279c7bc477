"""The bf16 grad_input against the packed state (rk_grad_input_bf16, the lm_head's backward):
out = bf16(G @ E), E = bf16(bf16(code) * bf16(scale)[:, None]) (ratchet.py:136-141), E
decoded into a workspace in MFMA operand order by the first of its two kernels.

Pinned two ways: bit for bit on inputs whose every partial sum is exactly representable
(small integer gradients, power-of-two scales: every summation order gives the exact sum,
so the result must equal torch's CPU product rounded once to bf16), and within the bf16
tolerance of north_star (rel 1e-2 of each element plus 1e-3 of the output's scale) on
realistic inputs, against float64 on the CPU. The effective weight itself is checked against
rk_effective_bf16, which restates the reference's two roundings.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import synthetic_state
from local_ai_training import _native as nat
from local_ai_training.int8_matmul import (effective_bf16, grad_input_bf16,
                                           grad_input_bf16_supported)

pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


def _code(packed, mc):
    return (packed.astype(np.int16) & 15) - mc


@pytest.mark.parametrize("m,n,k,mc", [(16384, 8192, 512, 2), (8192, 8192, 2048, 3),
                                      (1000, 96, 272, 7), (130, 32, 16, 1), (257, 4096, 144, 5),
                                      (77, 40, 32, 3), (300, 8, 784, 4)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_exact_sums_bit_for_bit(cuda, m, n, k, mc, out_dtype):
    packed, _ = synthetic_state(n, k, mc, seed=m + n + k)
    # power-of-two scales and small integer gradients: every partial sum is an integer
    # multiple of 2^-6 below 2^24 ulps, so every summation order gives the exact sum
    scale = (2.0 ** -torch.randint(0, 4, (n,), generator=gen(1)).float())
    g = torch.randint(-3, 4, (m, n), generator=gen(2)).to(torch.bfloat16)
    out = grad_input_bf16(g.to(cuda), torch.from_numpy(packed).to(cuda), mc, scale.to(cuda),
                          out_dtype)
    e = torch.from_numpy(_code(packed, mc)).double() * scale.double()[:, None]
    want = (g.double() @ e).to(torch.bfloat16)
    assert out.dtype == out_dtype
    assert torch.equal(out.cpu().to(torch.bfloat16).view(torch.int16), want.view(torch.int16))
    if out_dtype == torch.float32:
        assert torch.equal(out.cpu(), want.float())  # the bf16 value widened


@pytest.mark.parametrize("m,n,k,mc", [(16384, 8192, 512, 2), (8192, 8192, 2048, 3),
                                      (1000, 96, 272, 7)])
def test_realistic_inputs_within_the_bf16_tolerance(cuda, m, n, k, mc):
    packed, scale = synthetic_state(n, k, mc, seed=n + k)
    g = (torch.randn(m, n, generator=gen(3)) * 1e-2).to(torch.bfloat16)
    pd, sd = torch.from_numpy(packed).to(cuda), torch.from_numpy(scale).to(cuda)
    out = grad_input_bf16(g.to(cuda), pd, mc, sd).float().cpu()
    e = effective_bf16(pd, mc, sd).cpu()  # the reference's bf16(code) * bf16(scale)
    want = g.double() @ e.double()
    err = (out.double() - want).abs()
    assert bool((err <= 1e-2 * want.abs() + 1e-3 * want.abs().max()).all())
    # float reassociation only: nearly every element is the correctly rounded sum
    assert float((out == want.to(torch.bfloat16).float()).double().mean()) > 0.98


def test_strided_gradient_and_the_c_abi_checks(cuda):
    m, n, k, mc = 300, 256, 128, 3
    packed, scale = synthetic_state(n, k, mc, seed=9)
    big = torch.randint(-3, 4, (m, n + 64), generator=gen(4)).to(torch.bfloat16).to(cuda)
    g = big[:, 16:16 + n]  # row stride n + 64, 32-byte offset
    pd, sd = torch.from_numpy(packed).to(cuda), torch.ones(n, device=cuda)
    out = grad_input_bf16(g, pd, mc, sd)
    want = (g.cpu().double() @ torch.from_numpy(_code(packed, mc)).double()).to(torch.bfloat16)
    assert torch.equal(out.cpu().view(torch.int16), want.view(torch.int16))
    dst = torch.empty(m, k, dtype=torch.bfloat16, device=cuda)
    stream = nat.stream_handle(cuda)
    need = nat.load_library().rk_grad_input_bf16_workspace(n, k)
    assert need == 4 * 8 * 4096  # 4 steps of 64 rows x 8 blocks of 32 columns, 1 KB per sub-step
    work = torch.empty(need, dtype=torch.uint8, device=cuda)
    nat.call("rk_grad_input_bf16", g.data_ptr(), n + 64, pd.data_ptr(), k, mc, sd.data_ptr(),
             dst.data_ptr(), nat.RK_BF16, k, m, n, k, work.data_ptr(), need, stream)
    assert torch.equal(dst.cpu().view(torch.int16), want.view(torch.int16))
    with pytest.raises(nat.NativeError, match="workspace too small"):
        nat.call("rk_grad_input_bf16", g.data_ptr(), n + 64, pd.data_ptr(), k, mc, sd.data_ptr(),
                 dst.data_ptr(), nat.RK_BF16, k, m, n, k, work.data_ptr(), need - 16, stream)
    with pytest.raises(nat.NativeError, match="multiple of 8"):
        nat.call("rk_grad_input_bf16", g.data_ptr(), n + 64, pd.data_ptr(), k, mc, sd.data_ptr(),
                 dst.data_ptr(), nat.RK_BF16, k, m, 250, k, work.data_ptr(), need, stream)
    # the wrapper's gate matches the entry point's: packed rows of 264 bytes are not 16-byte
    # aligned, so that shape takes torch's GEMM on the effective weight instead
    p264 = torch.zeros(n, 264, dtype=torch.uint8, device=cuda)
    d264 = torch.empty(m, 264, dtype=torch.bfloat16, device=cuda)
    assert not grad_input_bf16_supported(g, p264) and grad_input_bf16_supported(g, pd)
    with pytest.raises(nat.NativeError, match="multiple of 8"):
        nat.call("rk_grad_input_bf16", g.data_ptr(), n + 64, p264.data_ptr(), 264, mc,
                 sd.data_ptr(), d264.data_ptr(), nat.RK_BF16, 264, m, n, 264, work.data_ptr(),
                 need, stream)
    with pytest.raises(nat.NativeError, match="max_code"):
        nat.call("rk_grad_input_bf16", g.data_ptr(), n + 64, pd.data_ptr(), k, 0, sd.data_ptr(),
                 dst.data_ptr(), nat.RK_BF16, k, m, n, k, work.data_ptr(), need, stream)


def test_model_lm_head_backward_uses_the_kernel(cuda):
    # A model step reaches the kernel through the lm_head (bf16 grad_input) and the layers
    # with int8_backward off; its input gradient equals torch's GEMM on the materialized
    # effective weight within the bf16 tolerance.
    from local_ai_training import ratchet

    calls = []
    orig = ratchet.grad_input_bf16

    def recording(*args, **kwargs):
        calls.append(args[0].shape)
        return orig(*args, **kwargs)

    ratchet.grad_input_bf16 = recording
    try:
        layer = ratchet.DiscreteRatchetLinear(512, 8192, max_code=2, matmul_mode="int8",
                                              fuse_backward_update=True).to(cuda).train()
        x = (torch.randn(256, 512, generator=gen(5))).to(cuda).requires_grad_(True)
        gout = (torch.randn(256, 8192, generator=gen(6)) * 1e-2).to(cuda)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = layer(x)
        packed0 = layer.packed.clone()
        out.backward(gout)
    finally:
        ratchet.grad_input_bf16 = orig
    assert calls == [(256, 8192)]
    e = effective_bf16(packed0, 2, layer.scale.detach()).float()
    want = gout.to(torch.bfloat16).float() @ e
    got = x.grad.float()
    assert bool(((got - want).abs() <= 1e-2 * want.abs() + 1e-3 * want.abs().max()).all())
