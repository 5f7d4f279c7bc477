"""Backward of the RMSNorm and tanh-GELU prologues on the GPU (rk_rmsnorm_backward,
rk_gelu_backward) against float64 autograd of the forward functions on the CPU.

The reference kernels (int8_backward.py:7-89) restate the analytic derivatives of
``x * rsqrt(mean(x^2) + eps) * w`` and of the tanh-GELU; autograd of those forwards in
float64 fixes the same quantities independently of the restated formulas. Tolerances:
grad_x is rounded to bf16 (relative step 2^-8), checked at rel 1e-2 / abs 1e-3 of the
gradient scale; grad_w is a float32 sum over rows, checked at 1e-5 of the sum of
absolute terms per column.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from local_ai_training import _native as nat
from local_ai_training import ops
from local_ai_training.int8_backward import gelu_backward, rmsnorm_backward

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16]


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def _rms_reference(x: torch.Tensor, gy: torch.Tensor, w: torch.Tensor, eps: float):
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    y = F.rms_norm(xd, (x.shape[-1],), wd, eps)
    gx, gw = torch.autograd.grad(y, (xd, wd), gy.double())
    xf = x.double()
    rs = torch.rsqrt((xf * xf).mean(dim=-1, keepdim=True) + eps)
    gw_abs = (gy.double() * xf * rs).abs().reshape(-1, x.shape[-1]).sum(dim=0)
    return gx, gw, gw_abs


def _assert_bf16_valued(t: torch.Tensor) -> None:
    f = t.float()
    assert torch.equal(f, f.to(torch.bfloat16).float()), "grad_x is not bf16-rounded"


def _check_grad_x(got: torch.Tensor, want: torch.Tensor) -> None:
    got = got.double().cpu()
    scale = float(want.abs().max()) if want.numel() else 1.0
    err = (got - want).abs()
    bound = 1e-2 * want.abs() + 1e-3 * scale
    assert bool((err <= bound).all()), f"max err {float(err.max())} (scale {scale})"


@pytest.mark.parametrize("m,k", [(4096, 512), (300, 2048), (7, 300), (1, 5), (33, 4096),
                                 (64, 768), (0, 64)])
@pytest.mark.parametrize("x_dtype", DTYPES)
@pytest.mark.parametrize("g_dtype", DTYPES)
def test_rmsnorm_backward_matches_float64_autograd(cuda, m, k, x_dtype, g_dtype):
    gen = torch.Generator().manual_seed(m * 131 + k)
    x = (torch.randn(m, k, generator=gen) * 1.5 + 0.25).to(x_dtype)
    gy = torch.randn(m, k, generator=gen).to(g_dtype)
    w = torch.rand(k, generator=gen) * 1.5 + 0.25
    eps = 1e-5
    gx, gw = rmsnorm_backward(gy.to(cuda), x.to(cuda), w.to(cuda), eps)
    assert gx.dtype == x_dtype and gx.shape == x.shape
    assert gw.dtype == torch.float32 and gw.shape == (k,)
    _assert_bf16_valued(gx)
    want_gx, want_gw, gw_abs = _rms_reference(x, gy, w, eps)
    _check_grad_x(gx, want_gx)
    err = (gw.double().cpu() - want_gw).abs()
    assert bool((err <= 1e-5 * gw_abs + 1e-30).all()), float(err.max())


def test_rmsnorm_backward_strided_rows_and_3d_inputs(cuda):
    # Row stride 515 (not a multiple of 4) forces the element-wise path; [B, S, K]
    # inputs flatten to rows as in the reference (x.flatten(0, -2)).
    gen = torch.Generator().manual_seed(5)
    base = torch.randn(96, 515, generator=gen)
    x = base[:, 3:515]
    gy = torch.randn(96, 512, generator=gen)
    w = torch.rand(512, generator=gen) + 0.5
    x_dev = base.to(cuda)[:, 3:515]
    assert x_dev.stride(0) == 515
    gx, gw = rmsnorm_backward(gy.to(cuda), x_dev, w.to(cuda))
    want_gx, want_gw, gw_abs = _rms_reference(x, gy, w, 1e-5)
    _check_grad_x(gx, want_gx)
    assert bool(((gw.double().cpu() - want_gw).abs() <= 1e-5 * gw_abs).all())
    gx3, gw3 = rmsnorm_backward(gy.view(4, 24, 512).to(cuda), x.reshape(4, 24, 512).to(cuda),
                                w.to(cuda))
    assert gx3.shape == (4, 24, 512)
    assert torch.equal(gx3.reshape(96, 512).cpu(), gx.cpu())
    assert torch.equal(gw3.cpu(), gw.cpu())


def test_rmsnorm_backward_is_reproducible(cuda):
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(16384, 512, generator=gen).to(cuda)
    gy = (torch.randn(16384, 512, generator=gen) * 1e-2).to(torch.bfloat16).to(cuda)
    w = (torch.rand(512, generator=gen) + 0.5).to(cuda)
    a = rmsnorm_backward(gy, x, w)
    b = rmsnorm_backward(gy, x, w)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("m,k,g_dtype", [(16384, 512, torch.bfloat16), (300, 2048, torch.float32),
                                         (37, 200, torch.bfloat16), (8, 4096, torch.float32)])
def test_rmsnorm_backward_with_residual_gradient_equals_backward_then_add(cuda, m, k, g_dtype):
    # grad_x = bf16(dx) + residual_grad in the kernel's store: the same bits as the plain
    # backward followed by the float32 add autograd performs for a block input with two uses;
    # through the operator, and through the C ABI out of place and in place
    x = (torch.randn(m, k, generator=gen(m + k)) * 2.0).to(cuda)
    w = (torch.rand(k, generator=gen(3)) + 0.5).to(cuda)
    gy = (torch.randn(m, k, generator=gen(4)) * 1e-2).to(g_dtype).to(cuda)
    res = (torch.randn(m, k, generator=gen(5)) * 1e-2).to(cuda)
    gx0, gw0 = rmsnorm_backward(gy, x, w, 1e-5)
    want = gx0 + res
    gx1, gw1 = rmsnorm_backward(gy, x, w, 1e-5, residual_grad=res)
    assert torch.equal(gx1.view(torch.int32), want.view(torch.int32))
    assert torch.equal(gw1, gw0)
    parts = int(nat.load_library().rk_rmsnorm_backward_parts(m))
    work = torch.empty(parts, k, device=cuda)
    gw2 = torch.empty(k, device=cuda)
    out = torch.empty(m, k, device=cuda)
    gdt = nat.RK_F32 if g_dtype == torch.float32 else nat.RK_BF16
    args = (gy.data_ptr(), gdt, k, x.data_ptr(), k, w.data_ptr(), 1e-5, m, k)
    tail = (gw2.data_ptr(), work.data_ptr(), work.numel(), nat.stream_handle(cuda))
    nat.call("rk_rmsnorm_backward_residual", *args, res.data_ptr(), k, out.data_ptr(), k, *tail)
    inplace = res.clone()
    nat.call("rk_rmsnorm_backward_residual", *args, inplace.data_ptr(), k, inplace.data_ptr(),
             k, *tail)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), want.view(torch.int32))
    assert torch.equal(inplace.view(torch.int32), want.view(torch.int32))
    assert torch.equal(gw2, gw0)


def test_rmsnorm_backward_residual_rejects_partial_overlap_and_bf16_x(cuda):
    m, k = 64, 256
    x = torch.randn(m, k, device=cuda)
    w = torch.ones(k, device=cuda)
    gy = torch.randn(m, k, device=cuda)
    buf = torch.randn(m + 1, k, device=cuda)
    work = torch.empty(int(nat.load_library().rk_rmsnorm_backward_parts(m)), k, device=cuda)
    gw = torch.empty(k, device=cuda)
    with pytest.raises(nat.NativeError, match="overlap"):
        nat.call("rk_rmsnorm_backward_residual", gy.data_ptr(), nat.RK_F32, k, x.data_ptr(), k,
                 w.data_ptr(), 1e-5, m, k, buf[1:].data_ptr(), k, buf[:-1].data_ptr(), k,
                 gw.data_ptr(), work.data_ptr(), work.numel(), nat.stream_handle(cuda))
    with pytest.raises(RuntimeError, match="float32 x"):
        ops.ratchet().rmsnorm_backward(gy, x.to(torch.bfloat16), w, 1e-5, gy)


def test_rmsnorm_backward_wide_rows_use_the_tensor_formulas(cuda):
    gen = torch.Generator().manual_seed(13)
    x = torch.randn(6, 4100, generator=gen)
    gy = torch.randn(6, 4100, generator=gen)
    w = torch.rand(4100, generator=gen) + 0.5
    gx, gw = rmsnorm_backward(gy.to(cuda), x.to(cuda), w.to(cuda))
    want_gx, want_gw, gw_abs = _rms_reference(x, gy, w, 1e-5)
    _check_grad_x(gx, want_gx)
    assert bool(((gw.double().cpu() - want_gw).abs() <= 1e-5 * gw_abs).all())


def _gelu_reference(x: torch.Tensor, gy: torch.Tensor) -> torch.Tensor:
    xd = x.double().requires_grad_(True)
    (gx,) = torch.autograd.grad(F.gelu(xd, approximate="tanh"), (xd,), gy.double())
    return gx


@pytest.mark.parametrize("m,k", [(4096, 2048), (129, 512), (5, 7), (1, 1), (3, 1030), (0, 16)])
@pytest.mark.parametrize("x_dtype", DTYPES)
@pytest.mark.parametrize("g_dtype", DTYPES)
def test_gelu_backward_matches_float64_autograd(cuda, m, k, x_dtype, g_dtype):
    gen = torch.Generator().manual_seed(m * 7 + k)
    x = (torch.randn(m, k, generator=gen) * 3.0).to(x_dtype)
    gy = torch.randn(m, k, generator=gen).to(g_dtype)
    gx = gelu_backward(gy.to(cuda), x.to(cuda))
    assert gx.dtype == x_dtype and gx.shape == x.shape
    _assert_bf16_valued(gx)
    _check_grad_x(gx, _gelu_reference(x, gy))


def test_gelu_backward_special_values(cuda):
    # Large |x| saturates tanh: the derivative tends to 1 (x >> 0) and 0 (x << 0);
    # at x = 0 it is exactly 0.5.
    x = torch.tensor([[0.0, 30.0, -30.0, 1e-20, -1e-20, 8.0, -8.0, 0.5]])
    gy = torch.ones_like(x)
    gx = gelu_backward(gy.to(cuda), x.to(cuda)).cpu()
    assert gx[0, 0] == 0.5
    assert gx[0, 1] == 1.0 and gx[0, 2] == 0.0
    _check_grad_x(gx, _gelu_reference(x, gy))


def test_gelu_backward_strided_rows(cuda):
    gen = torch.Generator().manual_seed(17)
    base = torch.randn(64, 2051, generator=gen)
    x = base[:, 1:2049]
    gy = torch.randn(64, 2048, generator=gen).to(torch.bfloat16)
    x_dev = base.to(cuda)[:, 1:2049]
    assert x_dev.stride(0) == 2051
    gx = gelu_backward(gy.to(cuda), x_dev)
    _check_grad_x(gx, _gelu_reference(x, gy))
