"""rk_grad_weight_bf16_noalloc: the allocation-free grad_weight entry point against the
workspace entry point rk_grad_weight_bf16, through the C ABI.

The split partials live in the library's file-scope device array, so the two entry points
run the same kernels in the same split order: with the same nsplit the bf16 results are
identical bit for bit. Two calls in a row, the second smaller (the array keeps the first
call's partials; the second must overwrite what it reads), then a call whose partials do
not fit is rejected. Free device memory does not move across the calls (no allocation).
"""

from __future__ import annotations

import pytest
import torch

from local_ai_training import _native as nat


def _grad_weight(cuda, m, n, k, g_dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    g = (torch.randn(m, n, generator=gen) * 1e-2).to(g_dtype).to(cuda)
    q = torch.randint(-127, 128, (m, k), generator=gen, dtype=torch.int8).to(cuda)
    s = (torch.rand(m, generator=gen) * 0.05 + 1e-3).to(cuda)
    nsplit = int(nat.load_library().rk_grad_weight_splits(m, n, k))
    return g, q, s, nsplit


def _dt(g):
    return nat.RK_F32 if g.dtype == torch.float32 else nat.RK_BF16


@pytest.mark.gpu
def test_noalloc_grad_weight_equals_the_workspace_entry_point_twice(cuda):
    stream = nat.stream_handle(cuda)
    cases = [(4096, 2048, 512, torch.bfloat16, 1), (1000, 512, 256, torch.float32, 2)]
    inputs = [_grad_weight(cuda, m, n, k, dt, seed) for m, n, k, dt, seed in cases]
    wants, gots = [], []
    for (m, n, k, _, _), (g, q, s, nsplit) in zip(cases, inputs):
        work = torch.empty(nsplit, n, k, dtype=torch.float32, device=cuda)
        want = torch.empty(n, k, dtype=torch.bfloat16, device=cuda)
        nat.call("rk_grad_weight_bf16", g.data_ptr(), _dt(g), n, q.data_ptr(), k, s.data_ptr(),
                 m, n, k, work.data_ptr(), nsplit, want.data_ptr(), k, stream)
        wants.append(want)
        gots.append(torch.full((n, k), float("nan"), dtype=torch.bfloat16, device=cuda))
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info(cuda)[0]
    for (m, n, k, _, _), (g, q, s, nsplit), got in zip(cases, inputs, gots):
        nat.call("rk_grad_weight_bf16_noalloc", g.data_ptr(), _dt(g), n, q.data_ptr(), k,
                 s.data_ptr(), m, n, k, nsplit, got.data_ptr(), k, stream)
        torch.cuda.synchronize()
    free_after = torch.cuda.mem_get_info(cuda)[0]
    for want, got in zip(wants, gots):
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert free_after == free_before


@pytest.mark.gpu
def test_noalloc_grad_weight_rejects_partials_beyond_the_scratch(cuda):
    m, n, k = 512, 4096, 4096  # 2 splits of 16 Mi floats: twice the scratch
    g = torch.zeros(m, n, dtype=torch.bfloat16, device=cuda)
    q = torch.zeros(m, k, dtype=torch.int8, device=cuda)
    s = torch.ones(m, device=cuda)
    out = torch.empty(n, k, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(nat.NativeError, match="exceed"):
        nat.call("rk_grad_weight_bf16_noalloc", g.data_ptr(), nat.RK_BF16, n, q.data_ptr(), k,
                 s.data_ptr(), m, n, k, 2, out.data_ptr(), k, nat.stream_handle(cuda))
    with pytest.raises(nat.NativeError, match="null output"):
        nat.call("rk_grad_weight_bf16_noalloc", g.data_ptr(), nat.RK_BF16, n, q.data_ptr(), k,
                 s.data_ptr(), m, n, k, 1, None, k, nat.stream_handle(cuda))
