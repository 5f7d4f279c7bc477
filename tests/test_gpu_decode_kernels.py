"""Fused decode kernels (rk_decode_gemv / rk_decode_attention / rk_decode_embed).

The GEMV's prologues reproduce the training quant kernels' arithmetic and its int32
sums and bf16 epilogue the packed GEMM's, so every GEMV output is compared bit for bit:
with the numpy oracle (per-token quant + scaled int8 GEMM) for int8/plain rows, and
with the HIP chain it replaces (rk_rmsnorm_quantize / rk_gelu_quantize +
rk_int8_gemm_packed) for the RMSNorm and GELU forms. The attention is float32 with a
split softmax: its rows are compared with a float64 softmax(q k^T / sqrt(D)) v on the
same keys at 2e-5 of each row's scale; the key/value append at `pos` is exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import synthetic_state
from local_ai_training import _native as nat
from local_ai_training.decode import (
    EPI_ADD,
    EPI_GELU,
    EPI_STORE,
    PRO_INT8,
    PRO_PLAIN,
    PRO_RMSNORM,
    attention_workspace_floats,
    decode_attention,
    decode_greedy,
)
from local_ai_training.int8_matmul import packed_int8_mm, quantize_rows
from oracle import gemm as ogemm
from oracle import quant as oquant

pytestmark = pytest.mark.gpu


class _Layer:
    """The attributes decode_gemv reads from a ratchet layer."""

    def __init__(self, packed, scale, max_code):
        self.packed, self.scale, self.max_code = packed, scale, max_code


def _layer(cuda, n, k, max_code, seed):
    packed, scale = synthetic_state(n, k, max_code, seed)
    return _Layer(torch.from_numpy(packed).to(cuda), torch.from_numpy(scale).to(cuda), max_code)


def _gemv(layer, out, prologue, epilogue, x=None, xq=None, xs=None, w=None, eps=0.0):
    from local_ai_training.decode import decode_gemv

    return decode_gemv(layer, out, prologue=prologue, epilogue=epilogue, x=x, xq=xq, xs=xs,
                       norm_weight=w, eps=eps)


# (1, 5632, 2048) and (1, 6144, 32): one token row over rows longer than 2048, the
# 8-wavefront split of K (the batch-1 contraction of the 1B model); (16, 2048, 6144) and
# (16, 2048, 8192): the 1B qkv and lm_head at batch 16 (two 16-row tiles per workgroup,
# as (12, 1024, 4096) with fewer token rows); (16, 2048, 2048), (16, 5632, 2048),
# (13, 2048, 2048), (9, 5632, 2048), (11, 6144, 32): groups of 8 token rows (the last one
# partial)
SHAPES = [(1, 2048, 6144), (1, 64, 16), (3, 2048, 5632), (4, 5632, 2048), (5, 320, 48),
          (16, 2048, 2048), (16, 5632, 2048), (11, 6144, 32), (1, 2048, 8192),
          (1, 5632, 2048), (1, 6144, 32), (16, 2048, 6144), (16, 2048, 8192),
          (12, 1024, 4096), (13, 2048, 2048), (9, 5632, 2048)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("max_code", [2, 3])
def test_plain_prologue_matches_the_oracle(cuda, m, k, n, max_code):
    gen = torch.Generator().manual_seed(m * 7 + k + n)
    x = torch.randn(m, k, generator=gen) * 3.0
    layer = _layer(cuda, n, k, max_code, seed=n + k)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=cuda)
    _gemv(layer, out, PRO_PLAIN, EPI_STORE, x=x.to(cuda))
    q, s = oquant.quantize_rows(x.numpy())
    code = ((layer.packed.cpu().numpy() & 15).astype(np.int16) - max_code).astype(np.int8)
    want = ogemm.scaled_int8_mm(q, code.T, s, layer.scale.cpu().numpy())  # bf16 bits
    assert np.array_equal(out.cpu().view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_int8_prologue_and_residual_add_match_the_packed_gemm(cuda, m, k, n):
    gen = torch.Generator().manual_seed(m + 3 * k + n)
    q = torch.randint(-127, 128, (m, k), generator=gen, dtype=torch.int8).to(cuda)
    s = (torch.rand(m, generator=gen) * 0.05 + 1e-3).to(cuda)
    layer = _layer(cuda, n, k, 3, seed=k + 1)
    residual = torch.randn(m, n, generator=gen).to(cuda)
    got = residual.clone()
    _gemv(layer, got, PRO_INT8, EPI_ADD, xq=q, xs=s)
    gemm = packed_int8_mm(q, layer.packed, 3, s, layer.scale, torch.float32)
    assert torch.equal(got, residual + gemm)
    stored = torch.empty(m, n, dtype=torch.float32, device=cuda)
    _gemv(layer, stored, PRO_INT8, EPI_STORE, xq=q, xs=s)
    assert torch.equal(stored, gemm)


@pytest.mark.parametrize("m,k,n", [(1, 2048, 6144), (4, 2048, 2048), (16, 2048, 5632),
                                   (7, 512, 128), (2, 5632, 64), (1, 5632, 64),
                                   (1, 6144, 128), (10, 6144, 64), (14, 2048, 4096)])
def test_rmsnorm_prologue_equals_rmsnorm_quantize_then_gemm(cuda, m, k, n):
    gen = torch.Generator().manual_seed(m + k + 5 * n)
    x = (torch.randn(m, k, generator=gen) * 2.0).to(cuda)
    w = (torch.rand(k, generator=gen) + 0.5).to(cuda)
    layer = _layer(cuda, n, k, 2, seed=n)
    got = torch.empty(m, n, dtype=torch.bfloat16, device=cuda)
    _gemv(layer, got, PRO_RMSNORM, EPI_STORE, x=x, w=w, eps=1e-5)
    q = torch.empty(m, k, dtype=torch.int8, device=cuda)
    s = torch.empty(m, dtype=torch.float32, device=cuda)
    nat.call("rk_rmsnorm_quantize", x.data_ptr(), nat.RK_F32, k, w.data_ptr(), 1e-5,
             q.data_ptr(), k, s.data_ptr(), m, k, nat.stream_handle(cuda))
    want = packed_int8_mm(q, layer.packed, 2, s, layer.scale, torch.bfloat16)
    assert torch.equal(got, want)


@pytest.mark.parametrize("m,k,n", [(1, 2048, 5632), (16, 2048, 5632), (3, 640, 96),
                                   (1, 5632, 128), (1, 6144, 64), (6, 1024, 4096),
                                   (15, 2048, 96)])
def test_gelu_epilogue_feeds_the_same_quantization_as_gelu_quantize(cuda, m, k, n):
    # expand GEMV with the GELU epilogue, then a plain quant of its float32 rows, must give
    # the q, s that rk_gelu_quantize computes from the GEMM's widened output
    gen = torch.Generator().manual_seed(m * k + n)
    q = torch.randint(-127, 128, (m, k), generator=gen, dtype=torch.int8).to(cuda)
    s = (torch.rand(m, generator=gen) * 0.05 + 1e-3).to(cuda)
    layer = _layer(cuda, n, k, 3, seed=9)
    gelu = torch.empty(m, n, dtype=torch.float32, device=cuda)
    _gemv(layer, gelu, PRO_INT8, EPI_GELU, xq=q, xs=s)
    expanded = packed_int8_mm(q, layer.packed, 3, s, layer.scale, torch.float32)
    qg = torch.empty(m, n, dtype=torch.int8, device=cuda)
    sg = torch.empty(m, dtype=torch.float32, device=cuda)
    nat.call("rk_gelu_quantize", expanded.data_ptr(), nat.RK_F32, n, qg.data_ptr(), n,
             sg.data_ptr(), m, n, nat.stream_handle(cuda))
    qd, sd = quantize_rows(gelu)
    assert torch.equal(qd, qg) and torch.equal(sd, sg)
    ref = torch.nn.functional.gelu(expanded.double(), approximate="tanh")
    assert float((gelu.double() - ref).abs().max()) <= 1e-5 * float(ref.abs().max()) + 1e-6


def test_decode_gemv_rejects_unsupported_shapes(cuda):
    layer = _layer(cuda, 40, 64, 2, seed=1)  # N % 16 != 0
    out = torch.empty(1, 40, dtype=torch.bfloat16, device=cuda)
    x = torch.zeros(1, 64, device=cuda)
    with pytest.raises(nat.NativeError, match="N % 16"):
        _gemv(layer, out, PRO_PLAIN, EPI_STORE, x=x)
    layer = _layer(cuda, 16, 64, 2, seed=1)
    out = torch.empty(17, 16, dtype=torch.float32, device=cuda)
    with pytest.raises(nat.NativeError, match="at most 16 rows"):
        _gemv(layer, out, PRO_PLAIN, EPI_STORE, x=torch.zeros(17, 64, device=cuda))
    out = torch.empty(1, 16, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(nat.NativeError, match="write float32"):
        _gemv(layer, out, PRO_PLAIN, EPI_ADD, x=x)
    rows = torch.zeros(1, 80, device=cuda)
    with pytest.raises(nat.NativeError, match="must not overlap"):
        _gemv(layer, rows[:, 48:64], PRO_PLAIN, EPI_ADD, x=rows[:, :64])
    _gemv(layer, rows[:, 64:], PRO_PLAIN, EPI_ADD, x=rows[:, :64])  # disjoint: accepted


def _attention_case(cuda, batch, heads, head, max_len, pos, cache_dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    c = heads * head
    # bf16-valued projections, as the qkv GEMV writes them
    qkv = (torch.randn(batch, 3 * c, generator=gen) * 2.0).to(torch.bfloat16).to(cuda)
    keys = (torch.randn(batch, heads, max_len, head, generator=gen)).to(cache_dtype).to(cuda)
    values = (torch.randn(batch, heads, max_len, head, generator=gen)).to(cache_dtype).to(cuda)
    return qkv, keys, values


@pytest.mark.parametrize("batch,heads,head,max_len,pos", [
    (1, 16, 128, 1024, 1023), (1, 16, 128, 1024, 0), (1, 16, 128, 1024, 600),
    (16, 16, 128, 1024, 959), (3, 4, 64, 64, 17), (2, 2, 256, 48, 47), (5, 8, 64, 100, 1),
    (8, 16, 64, 200, 150), (16, 8, 128, 64, 0)])
@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float32])
def test_decode_attention_matches_float64_softmax(cuda, batch, heads, head, max_len, pos,
                                                  cache_dtype):
    qkv, keys, values = _attention_case(cuda, batch, heads, head, max_len, pos, cache_dtype,
                                        seed=batch * 31 + pos)
    keys_before, values_before = keys.clone(), values.clone()
    c = heads * head
    work = torch.empty(attention_workspace_floats(batch, heads, head, max_len),
                       dtype=torch.float32, device=cuda)
    out = torch.empty(batch, c, dtype=torch.float32, device=cuda)
    position = torch.tensor([pos], dtype=torch.long, device=cuda)
    decode_attention(qkv, keys, values, position, heads, work, out)
    torch.cuda.synchronize()
    # the append: position pos holds the step's k, v; every other position is untouched
    k_new = qkv[:, c:2 * c].view(batch, heads, head).to(cache_dtype)
    v_new = qkv[:, 2 * c:].view(batch, heads, head).to(cache_dtype)
    assert torch.equal(keys[:, :, pos], k_new) and torch.equal(values[:, :, pos], v_new)
    others = torch.ones(max_len, dtype=torch.bool)
    others[pos] = False
    assert torch.equal(keys[:, :, others], keys_before[:, :, others])
    assert torch.equal(values[:, :, others], values_before[:, :, others])
    # float64 reference over positions 0..pos (the keys hold bf16-exact values)
    q = qkv[:, :c].view(batch, heads, 1, head).double()
    k = keys[:, :, :pos + 1].double()
    v = values[:, :, :pos + 1].double()
    att = torch.softmax((q @ k.transpose(-1, -2)) / math.sqrt(head), dim=-1) @ v
    rows = att.view(batch, c)
    err = (out.double() - rows).abs().amax(dim=1) / rows.abs().amax(dim=1)
    assert float(err.max()) <= 2e-5


@pytest.mark.parametrize("batch,heads", [(2, 4), (16, 8)])
def test_decode_attention_out_of_range_position_touches_nothing(cuda, batch, heads):
    qkv, keys, values = _attention_case(cuda, batch, heads, 64, 32, 0, torch.bfloat16, seed=3)
    keys_before, values_before = keys.clone(), values.clone()
    work = torch.zeros(attention_workspace_floats(batch, heads, 64, 32), dtype=torch.float32,
                       device=cuda)
    out = torch.empty(batch, heads * 64, dtype=torch.float32, device=cuda)
    decode_attention(qkv, keys, values, torch.tensor([32], device=cuda), heads, work, out)
    torch.cuda.synchronize()
    assert torch.equal(keys, keys_before) and torch.equal(values, values_before)
    assert bool(torch.isnan(out).all())


def test_decode_attention_rejects_a_short_workspace(cuda):
    qkv, keys, values = _attention_case(cuda, 1, 4, 64, 32, 0, torch.bfloat16, seed=4)
    work = torch.empty(8, dtype=torch.float32, device=cuda)
    out = torch.empty(1, 256, dtype=torch.float32, device=cuda)
    with pytest.raises(nat.NativeError, match="workspace too small"):
        decode_attention(qkv, keys, values, torch.tensor([0], device=cuda), 4, work, out)


# (5, 1000, 24): float4 pieces of padded rows; (4, 1001, 0) and (3, 1, 3): scalar loads
@pytest.mark.parametrize("batch,vocab,pad", [(1, 8192, 0), (16, 8192, 0), (5, 1000, 24),
                                             (4, 1001, 0), (3, 1, 3), (2, 70000, 0)])
def test_decode_greedy_picks_the_first_argmax_and_advances(cuda, batch, vocab, pad):
    gen = torch.Generator().manual_seed(batch * 7 + vocab)
    rows = torch.randn(batch, vocab + pad, generator=gen)
    rows[:, vocab:] = 1e30  # padding past V is never read
    if vocab > 10:
        rows[0, 3] = rows[0, 7] = rows[0, :vocab].max() + 1.0  # a tie: the first index
        if batch > 1:
            rows[1, vocab - 2] = float("nan")  # a NaN ranks above every number
            rows[1, 5] = float("inf")
        if batch > 2:
            rows[2, :vocab] = float("-inf")  # all -inf: index 0
        if batch > 3:
            rows[3, 9] = rows[3, 4] = float("nan")  # the first NaN
    logits = rows.to(cuda)[:, :vocab]
    tokens = torch.full((batch, 2), -5, dtype=torch.long, device=cuda)
    pos = torch.tensor([41], dtype=torch.long, device=cuda)
    decode_greedy(logits, tokens[:, :1], pos)
    torch.cuda.synchronize()
    want = np.argmax(rows[:, :vocab].numpy(), axis=1)  # numpy: first max, NaN above all
    assert torch.equal(torch.argmax(rows[:, :vocab], dim=-1), torch.from_numpy(want))
    assert np.array_equal(tokens[:, 0].cpu().numpy(), want)
    assert bool((tokens[:, 1] == -5).all()) and int(pos) == 42
    decode_greedy(logits, tokens[:, 1:], None)  # no position: only the picks
    torch.cuda.synchronize()
    assert np.array_equal(tokens[:, 1].cpu().numpy(), want) and int(pos) == 42


# width 256: float4 pieces; 250: rows not 16-byte aligned, one element per thread; 4100:
# more than one pass of pieces per thread
@pytest.mark.parametrize("width", [256, 250, 4100])
def test_decode_embed_is_the_table_row_plus_the_position_row(cuda, width):
    gen = torch.Generator().manual_seed(2)
    table = torch.randn(300, width, generator=gen).to(cuda)
    positions = torch.randn(64, width, generator=gen).to(cuda)
    tokens = torch.tensor([5, 299, 0, 17], device=cuda)
    hidden = torch.empty(4, width, device=cuda)
    for p in (0, 63, 64):
        pos = torch.tensor([p], device=cuda)
        nat.call("rk_decode_embed", tokens.data_ptr(), 4, table.data_ptr(), 300, width,
                 positions.data_ptr(), 64, pos.data_ptr(), hidden.data_ptr(), width,
                 nat.stream_handle(cuda))
        torch.cuda.synchronize()
        if p < 64:
            assert torch.equal(hidden, table[tokens] + positions[p])
        else:
            assert bool(torch.isnan(hidden).all())
    bad = torch.tensor([300], device=cuda)
    nat.call("rk_decode_embed", bad.data_ptr(), 1, table.data_ptr(), 300, width,
             positions.data_ptr(), 64, torch.tensor([0], device=cuda).data_ptr(),
             hidden.data_ptr(), width, nat.stream_handle(cuda))
    torch.cuda.synchronize()
    assert bool(torch.isnan(hidden[0]).all())
