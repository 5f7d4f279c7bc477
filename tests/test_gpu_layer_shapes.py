"""Every distinct ratchet-layer shape of the 25M and 1B training configs, at full M.

25M (M = 16384 tokens = batch 32 x seq 512, quinary codes): qkv 1536x512, projection
512x512, expand 2048x512, contraction 512x2048, lm_head 8192x512.
1B (M = 8192 tokens = batch 8 x seq 1024, septenary codes): qkv 6144x2048, projection
2048x2048, expand 5632x2048, contraction 2048x5632, lm_head 8192x2048.

Each shape runs the layer's whole int8 step through the torch.ops.ratchet operators the
training path calls: per-token quant of bf16 N(0,1) activations, forward GEMM on the packed
state (float32 output), SR quant of a bf16 N(0, 1e-2) upstream gradient folded with the row
scales, int8 grad_input on the packed state, BF16 grad_weight split partials and the fused
update from them. Sampled rows (first and last included) are replayed by the oracle: bit
for bit for the quantized values, scales, GEMM outputs and the updated state (the update
consumes the bf16 gradient the GPU formed: shared producer); the bf16 grad_weight against a
float32 product at rel 1e-2 / abs 1e-3.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import synthetic_state
from local_ai_training.ops import ratchet
from oracle import quant as oquant
from oracle import update as oupd
from parity import (
    check_forward,
    check_grad_input,
    check_sr_quant,
    check_update,
    f32bits,
    sample_rows,
)

pytestmark = pytest.mark.gpu

SHAPES = [
    # name, tokens M, out N, in K, max_code
    ("25M-qkv", 16384, 1536, 512, 2),
    ("25M-proj", 16384, 512, 512, 2),
    ("25M-expand", 16384, 2048, 512, 2),
    ("25M-contract", 16384, 512, 2048, 2),
    ("25M-lm_head", 16384, 8192, 512, 2),
    ("1B-qkv", 8192, 6144, 2048, 3),
    ("1B-proj", 8192, 2048, 2048, 3),
    ("1B-expand", 8192, 5632, 2048, 3),
    ("1B-contract", 8192, 2048, 5632, 3),
    ("1B-lm_head", 8192, 8192, 2048, 3),
]


@pytest.mark.parametrize("name,m,n,k,mc", SHAPES, ids=[s[0] for s in SHAPES])
def test_layer_step_matches_oracle_on_sampled_rows(cuda, name, m, n, k, mc):
    print(f"layer shape {name}: M={m} N={n} K={k} max_code={mc}", flush=True)
    ops = ratchet()
    seed = sum(map(ord, name))
    cgen = torch.Generator(device=cuda).manual_seed(seed)
    x = torch.randn(m, k, generator=cgen, device=cuda).to(torch.bfloat16)
    g = (torch.randn(m, n, generator=cgen, device=cuda) * 1e-2).to(torch.bfloat16)
    packed_np, scale_np = synthetic_state(n, k, mc, seed=seed)
    packed = torch.from_numpy(packed_np).to(cuda)
    scale = torch.from_numpy(scale_np).to(cuda)
    rows = sample_rows(m, 48, seed)
    rows_t = torch.from_numpy(rows).to(cuda)
    out_rows = sample_rows(n, 48, seed + 1)
    code, _ = oupd.unpack(packed_np, mc)

    # per-token quant of the activations (A1)
    q, s = ops.quantize_rows(x)
    q_ref, s_ref = oquant.quantize_rows(x[rows_t].float().cpu().numpy())
    assert np.array_equal(q[rows_t].cpu().numpy(), q_ref)
    assert np.array_equal(f32bits(s[rows_t]), f32bits(s_ref))

    # forward GEMM on the packed state, float32 output (A3, A4)
    out = ops.packed_mm(q, packed, mc, s, scale, torch.float32)
    check_forward(code, scale_np, q[rows_t], s[rows_t], out[rows_t], what=name)
    del out

    # SR quant of the upstream gradient with the row scales folded in (A6)
    sr_seed = 1000 + seed
    gq, gs = ops.quantize_rows(g, scale, True, sr_seed)
    check_sr_quant(g[rows_t], scale_np, sr_seed, rows, gq[rows_t], gs[rows_t], what=name)

    # int8 grad_input on the packed state in place (A7)
    gin = ops.packed_mm_t(gq, packed, mc, gs, None, torch.bfloat16)
    check_grad_input(code, gq[rows_t], gs[rows_t], gin[rows_t], what=name)
    del gin, gq

    # BF16 grad_weight split partials (A9), the fused update from them (A10-A12)
    nsplit = ops.grad_weight_splits(m, n, k)
    work = torch.empty(nsplit, n, k, device=cuda)
    ops.grad_weight_partials(g, q, s, work)
    counts = torch.zeros(4, dtype=torch.int64, device=cuda)
    row_rms = torch.empty(n, device=cuda)
    flag = torch.zeros(1, dtype=torch.int32, device=cuda)
    kept = torch.empty(n, k, dtype=torch.bfloat16, device=cuda)
    ops.update_from_partials(packed, work, mc, 8, 0.5, 1.5, 1e-8, None, 0.0, counts, row_rms,
                             None, flag, None, kept)
    out_t = torch.from_numpy(out_rows).to(cuda)
    got = packed[out_t].cpu().numpy()
    moves = check_update(packed_np[out_rows], kept[out_t], got, mc, what=name)
    assert int(flag.item()) == 0

    xhat = (q.to(torch.bfloat16) * s.to(torch.bfloat16)[:, None]).float()
    want = g[:, out_t].float().t() @ xhat
    torch.testing.assert_close(kept[out_t].float(), want, rtol=1e-2, atol=1e-3)
    total = counts.cpu().numpy()
    assert total.sum() >= moves.sum()
    print(f"  {name}: ok (sampled moves {moves.tolist()}, all moves {total.tolist()})",
          flush=True)
