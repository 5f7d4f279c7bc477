"""grad_weight with the update in its last blocks (rk_grad_weight_update) against the two
launches it replaces: the grad_weight partials (rk_grad_weight_bf16 / _x with no output),
then rk_ratchet_update_partials over them. Same inputs, same split count, so every output
must be identical bit for bit: the packed state, the four move counts, row rms, the rms EMA,
the non-finite flag, the row rms mean and the kept bf16 gradient.

Shapes cover both tile configurations (128 x 128 and 256 x 256 output tiles), rows of one
register chunk (K <= 512) and streamed rows (K > 512), ragged row blocks and column tiles,
one split and many, the three activation forms, a float32 and a bf16 upstream gradient, and
a row with a non-finite gradient. Each case runs the fused call twice on the same arrival
counters (the second on new data): the counters must come back to zero after each call.
"""

from __future__ import annotations

import pytest
import torch

from local_ai_training import _native as nat

from helpers import synthetic_state


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def _inputs(m, n, k, mc, x_kind, g_dtype, seed, bad_row=None):
    g0 = gen(seed)
    g = torch.randn(m, n, generator=g0) * 1e-2
    if bad_row is not None:
        g[5, bad_row] = float("inf")  # column bad_row of the gradient: weight row bad_row
    g = g.to(g_dtype)
    q = torch.randint(-127, 128, (m, k), generator=g0, dtype=torch.int8)
    s = torch.rand(m, generator=g0) * 0.05 + 1e-3
    if x_kind == nat.RK_I8:
        x, xs = q, s
    else:
        x = (torch.randn(m, k, generator=g0)).to(torch.float32 if x_kind == nat.RK_F32
                                                 else torch.bfloat16)
        xs = None
    packed, _ = synthetic_state(n, k, mc, seed=seed + 1)
    return g, x, xs, torch.from_numpy(packed)


def _outputs(cuda, n, k, packed):
    return dict(packed=packed.clone().to(cuda), ema=torch.full((n,), 0.25, device=cuda),
                counts=torch.zeros(4, dtype=torch.int64, device=cuda),
                row_rms=torch.empty(n, device=cuda), flag=torch.zeros(1, dtype=torch.int32,
                                                                        device=cuda),
                mean=torch.empty((), device=cuda),
                kept=torch.zeros(n, k, dtype=torch.bfloat16, device=cuda))


def _dt(t):
    return nat.RK_F32 if t.dtype == torch.float32 else nat.RK_BF16


def _run(cuda, m, n, k, mc, g, x, xs, packed, nsplit, counters, fused):
    o = _outputs(cuda, n, k, packed)
    beta = 0.9
    stream = nat.stream_handle(cuda)
    work = torch.empty(nsplit, n, k, device=cuda)
    x_kind = nat.RK_I8 if x.dtype == torch.int8 else _dt(x)
    tail = (o["packed"].data_ptr(), k, mc, 8, 0.5, 1.5, 1e-8, o["ema"].data_ptr(), beta,
            1.0 - beta, o["counts"].data_ptr(), o["row_rms"].data_ptr())
    if fused:
        nat.call("rk_grad_weight_update", g.data_ptr(), _dt(g), n, x.data_ptr(), x_kind, k,
                 nat.ptr(xs), m, n, k, work.data_ptr(), nsplit, counters.data_ptr(), *tail,
                 o["flag"].data_ptr(), o["mean"].data_ptr(), o["kept"].data_ptr(), k, stream)
    else:
        if x_kind == nat.RK_I8:
            nat.call("rk_grad_weight_bf16", g.data_ptr(), _dt(g), n, x.data_ptr(), k,
                     xs.data_ptr(), m, n, k, work.data_ptr(), nsplit, None, k, stream)
        else:
            nat.call("rk_grad_weight_bf16_x", g.data_ptr(), _dt(g), n, x.data_ptr(), x_kind,
                     k, m, n, k, work.data_ptr(), nsplit, None, k, stream)
        nat.call("rk_ratchet_update_partials", o["packed"].data_ptr(), k, work.data_ptr(),
                 nsplit, n, k, mc, 8, 0.5, 1.5, 1e-8, o["ema"].data_ptr(), beta, 1.0 - beta,
                 o["counts"].data_ptr(), o["row_rms"].data_ptr(), None, o["flag"].data_ptr(),
                 o["mean"].data_ptr(), o["kept"].data_ptr(), k, stream)
    torch.cuda.synchronize()
    return o


def _same_bits(a, b):
    if a.dtype == torch.bfloat16:
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    if a.dtype in (torch.float32,):
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)


CASES = [
    # (M, N, K, nsplit or None = default, x form, g dtype, bad row)
    (16384, 2048, 512, None, nat.RK_I8, torch.bfloat16, None),   # op shape, small tiles
    (16384, 512, 2048, None, nat.RK_I8, torch.float32, 7),       # streamed rows
    (1024, 8192, 512, None, nat.RK_I8, torch.float32, None),     # 256 x 256 tiles, one chunk
    (2048, 4096, 2048, None, nat.RK_I8, torch.float32, None),    # 256 x 256 tiles, streamed
    (1024, 2048, 5632, 1, nat.RK_I8, torch.bfloat16, 300),       # one split, long rows
    (1000, 200, 144, 3, nat.RK_BF16, torch.bfloat16, None),      # ragged row / column tiles
    (640, 264, 1040, 5, nat.RK_F32, torch.float32, 263),         # ragged, float32 activations
]


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,nsplit,x_kind,g_dtype,bad", CASES)
def test_fused_grad_weight_update_equals_partials_then_update(cuda, m, n, k, nsplit, x_kind,
                                                              g_dtype, bad):
    mc = 3
    if nsplit is None:
        nsplit = int(nat.load_library().rk_grad_weight_splits(m, n, k))
    ncount = int(nat.load_library().rk_grad_weight_update_counters(n, k))
    counters = torch.zeros(ncount, dtype=torch.int32, device=cuda)
    for call in range(2):
        g, x, xs, packed = _inputs(m, n, k, mc, x_kind, g_dtype, seed=m + n + k + call,
                                   bad_row=bad)
        g, x = g.to(cuda), x.to(cuda)
        xs = xs.to(cuda) if xs is not None else None
        want = _run(cuda, m, n, k, mc, g, x, xs, packed, nsplit, counters, fused=False)
        got = _run(cuda, m, n, k, mc, g, x, xs, packed, nsplit, counters, fused=True)
        assert int(counters.abs().sum()) == 0, "arrival counters not reset"
        assert torch.equal(got["packed"], want["packed"])
        assert torch.equal(got["counts"], want["counts"])
        assert torch.equal(got["flag"], want["flag"])
        finite = torch.isfinite(want["row_rms"])
        for key in ("row_rms", "ema"):
            assert _same_bits(got[key][finite], want[key][finite]), key
        assert _same_bits(got["mean"], want["mean"]) or bool(want["mean"].isnan())
        ok = torch.isfinite(want["kept"].float()).all(dim=1)
        assert _same_bits(got["kept"][ok], want["kept"][ok])
        if bad is not None:
            assert int(got["flag"].item()) == 1
        assert int(want["counts"][:2].sum()) > 0  # the update moved codes


@pytest.mark.gpu
def test_fused_grad_weight_update_rejects_bad_arguments(cuda):
    n, k, m = 64, 60, 32  # K % 8 != 0
    g = torch.zeros(m, n, device=cuda)
    x = torch.zeros(m, k, dtype=torch.bfloat16, device=cuda)
    packed = torch.zeros(n, k, dtype=torch.uint8, device=cuda)
    counters = torch.zeros(4, dtype=torch.int32, device=cuda)
    work = torch.empty(1, n, k, device=cuda)
    with pytest.raises(nat.NativeError):
        nat.call("rk_grad_weight_update", g.data_ptr(), nat.RK_F32, n, x.data_ptr(),
                 nat.RK_BF16, k, None, m, n, k, work.data_ptr(), 1, counters.data_ptr(),
                 packed.data_ptr(), k, 2, 8, 0.5, 1.5, 1e-8, None, 0.0, 1.0, None, None, None,
                 None, None, k, nat.stream_handle(cuda))
    with pytest.raises(nat.NativeError, match="counters"):
        nat.call("rk_grad_weight_update", g.data_ptr(), nat.RK_F32, n, x.data_ptr(),
                 nat.RK_BF16, 64, None, m, n, 64, work.data_ptr(), 1, None,
                 packed.data_ptr(), 64, 2, 8, 0.5, 1.5, 1e-8, None, 0.0, 1.0, None, None, None,
                 None, None, 64, nat.stream_handle(cuda))
