"""Kernel-level parity: every HIP entry point against the numpy oracle, bit for bit.

Integer / byte / index outputs (int8 codes, int32 accumulators, packed bytes, move
counts) and the IEEE-defined float outputs (quant scales, bf16 GEMM outputs, row rms,
normalized gradients) must be identical. Inputs are seeded; shapes cover the reference
tests' ragged cases, the BASELINE op shape (M=16384, K=512, N=2048) and 1B-class rows.
"""

from __future__ import annotations

import math
import numpy as np
import pytest
import torch

from helpers import synthetic_state
from local_ai_training import _native as nat
from local_ai_training.ops import ratchet as ops
from local_ai_training.int8_matmul import (
    dequant_bf16,
    dequant_transpose_bf16,
    effective_bf16,
    grad_weight_bf16,
    grad_weight_bf16_parts,
    grad_weight_bf16_x,
    int8_mm_nt,
    packed_int8_mm,
    quantize_columns,
    quantize_rows,
    quantize_rows_colscaled,
    scaled_int8_mm,
    transpose_bf16,
    unpack_transpose,
)
from oracle import gemm as ogemm
from oracle import quant as oquant
from oracle import update as oupd
from oracle.numerics import f32_to_bf16_bits, round_to_bf16

pytestmark = pytest.mark.gpu


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def f32bits(a) -> np.ndarray:
    a = a.cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------------------
# Row quantization
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(67, 35), (128, 256), (1, 513), (255, 1), (300, 2048),
                                   (7, 5632), (16384, 512)])
def test_quantize_rows_bit_exact(cuda, shape, dtype):
    values = (torch.randn(shape, generator=gen(7)) * 3.0).to(dtype)
    q, s = quantize_rows(values.to(cuda))
    q_ref, s_ref = oquant.quantize_rows(values.float().numpy())
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(f32bits(s), f32bits(s_ref))


def test_quantize_rows_noncontiguous_and_zero_rows(cuda):
    base = (torch.randn(70, 48, generator=gen(11)) * 2.0).to(torch.bfloat16)
    view = base.to(cuda).t()
    q, s = quantize_rows(view)
    q_ref, s_ref = oquant.quantize_rows(base.t().float().numpy())
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(f32bits(s), f32bits(s_ref))
    zq, zs = quantize_rows(torch.zeros(3, 5, device=cuda, dtype=torch.bfloat16))
    assert int(torch.count_nonzero(zq)) == 0
    assert torch.all(zs == torch.finfo(torch.float32).tiny)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(67, 35), (128, 256), (1, 255), (300, 1), (64, 2048)])
def test_quantize_rows_colscaled_bit_exact(cuda, shape, dtype):
    g = (torch.randn(shape, generator=gen(21)) * 3.0).to(dtype)
    col = torch.rand(shape[1], generator=gen(22)) + 0.01
    q, s = quantize_rows_colscaled(g.to(cuda), col.to(cuda))
    q_ref, s_ref = oquant.quantize_rows(g.float().numpy(), col.numpy())
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(f32bits(s), f32bits(s_ref))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(8, 64), (67, 35), (33, 2048), (3, 5632)])
def test_stochastic_rounding_bit_exact_given_seed(cuda, shape, dtype):
    g = (torch.randn(shape, generator=gen(31)) * 1e-2).to(dtype)
    col = torch.rand(shape[1], generator=gen(32)) * 0.08 + 0.02
    gd = g.to(cuda)
    for seed in (0, 1, 123456789, 2**31 - 2):
        q, s = ops().quantize_rows(gd, col.to(cuda), True, seed)
        q_ref, s_ref = oquant.quantize_rows_sr(g.float().numpy(), col.numpy(), seed)
        assert np.array_equal(q.cpu().numpy(), q_ref), f"seed {seed}"
        assert np.array_equal(f32bits(s), f32bits(s_ref))


def philox_words(cuda, seed: int, counter0: int, n: int) -> np.ndarray:
    out = torch.empty(n, dtype=torch.int32, device=cuda)
    nat.call("rk_philox_word0", seed, counter0, n, out.data_ptr(), nat.stream_handle(cuda))
    return out.cpu().numpy().view(np.uint32)


def test_philox_words_match_random123_kat_and_oracle(cuda, golden):
    # Random123 KAT: counter 0, key 0 -> first word 6627e8d5 (the only published vector
    # whose counter has the (x, 0, 0, 0) form the stochastic rounding uses).
    kat = golden["philox4x32_10"]["vectors"][0]
    assert kat["ctr"] == ["00000000"] * 4 and kat["key"] == ["00000000"] * 2
    assert philox_words(cuda, 0, 0, 1)[0] == int(kat["out"][0], 16)
    from oracle import philox as ophilox
    for seed, c0, n in ((0, 0, 4096), (1234567, 17, 100_003), (2**31 - 2, 2**32 - 5000, 10_000),
                        ((7 << 32) | 99, 123, 50_000)):
        got = philox_words(cuda, seed, c0, n)
        offsets = (np.arange(n, dtype=np.uint64) + np.uint64(c0)) & np.uint64(0xFFFFFFFF)
        ref = ophilox.randint(seed, offsets.astype(np.uint32))
        assert np.array_equal(got, ref), f"seed {seed} counter0 {c0}"


def near_boundary_rows(rows: int, cols: int, seed: int, sr_seed: int | None):
    """Rows whose quotients x / s sit on or within a few ulps of the rounding boundaries
    (half-integers for rint; for SR, the integers minus the element's own uniform u), so
    the kernels' reciprocal fast path must defer to the IEEE division."""
    from oracle import philox as ophilox
    rng = np.random.default_rng(seed)
    amax = rng.uniform(0.5, 3.0, size=rows).astype(np.float32)
    s = np.maximum(amax / np.float32(127.0), np.float32(np.finfo(np.float32).tiny))
    k = rng.integers(-126, 126, size=(rows, cols)).astype(np.float32)
    if sr_seed is None:
        target = k + np.float32(0.5)
    else:
        u = ophilox.rand(sr_seed, ophilox.sr_offsets(rows, cols)).reshape(rows, cols)
        target = k - u
    x = (target * s[:, None]).astype(np.float32)
    ulps = rng.integers(-3, 4, size=(rows, cols)).astype(np.int32)
    x = (x.view(np.int32) + ulps).view(np.float32)
    x[:, 0] = amax  # pins the row absmax, so s is exactly amax / 127
    x[:, 1] = -amax
    return np.clip(x, -amax[:, None], amax[:, None])


@pytest.mark.parametrize("rows,cols", [(64, 512), (5, 2048), (33, 40)])
def test_quantize_rows_near_half_integer_quotients(cuda, rows, cols):
    x = near_boundary_rows(rows, cols, 3, None)
    q, s = quantize_rows(torch.from_numpy(x).to(cuda))
    q_ref, s_ref = oquant.quantize_rows(x)
    assert np.array_equal(f32bits(s), f32bits(s_ref))
    assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("rows,cols", [(64, 512), (5, 2048), (33, 40)])
def test_stochastic_rounding_near_integer_sums(cuda, rows, cols):
    seed = 4242
    x = near_boundary_rows(rows, cols, 5, seed)
    q, s = ops().quantize_rows(torch.from_numpy(x).to(cuda), None, True, seed)
    q_ref, s_ref = oquant.quantize_rows_sr(x, None, seed)
    assert np.array_equal(f32bits(s), f32bits(s_ref))
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_public_sr_draws_its_seed_from_the_cpu_generator(cuda):
    # int8_matmul.py:200: one torch.randint draw per stochastic call.
    g = torch.randn(16, 96, generator=gen(41))
    col = torch.rand(96, generator=gen(42)) + 0.01
    torch.manual_seed(5)
    seed = int(torch.randint(0, 2**31 - 1, (1,)).item())
    after_ref = torch.rand(3)
    torch.manual_seed(5)
    q, _ = quantize_rows_colscaled(g.to(cuda), col.to(cuda), stochastic=True)
    assert torch.equal(torch.rand(3), after_ref)  # CPU RNG stream advanced identically
    q_ref, _ = oquant.quantize_rows_sr(g.numpy(), col.numpy(), seed)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_sr_quant_full_op_shape_sampled_rows_and_bf16_side_output(cuda):
    m, n = 16384, 2048
    g = (torch.randn(m, n, generator=gen(51)) * 1e-2).to(torch.bfloat16)
    col = torch.rand(n, generator=gen(52)) * 0.08 + 0.02
    gd = g.to(cuda)
    side = torch.empty(m, n, dtype=torch.bfloat16, device=cuda)
    q, s = ops().quantize_rows(gd, col.to(cuda), True, 987654, x_bf16=side)
    assert torch.equal(side, gd)
    qc, sc = q.cpu().numpy(), s.cpu().numpy()
    rows = np.random.default_rng(0).choice(m, 256, replace=False)
    for r0 in rows:
        q_ref, s_ref = oquant.quantize_rows_sr(g[r0:r0 + 1].float().numpy(), col.numpy(),
                                               987654, row_start=int(r0))
        assert np.array_equal(qc[r0:r0 + 1], q_ref) and sc[r0] == s_ref[0]


def test_f32_gradient_side_output_is_rne_bf16(cuda):
    g = torch.randn(64, 512, generator=gen(53))
    side = torch.empty(64, 512, dtype=torch.bfloat16, device=cuda)
    ops().quantize_rows(g.to(cuda), None, True, 3, x_bf16=side)
    assert np.array_equal(bits16(side), f32_to_bf16_bits(g.numpy()))


@pytest.mark.parametrize("shape,strided", [((16384, 512), False), ((67, 35), False),
                                            ((33, 2048), True), ((9, 6144), False),
                                            ((5, 5632), True)])
def test_sr_quant_of_float32_as_bf16_equals_cast_then_quant(cuda, shape, strided):
    # round_bf16 (C ABI: RK_F32_AS_BF16) quantizes float32 values as their bf16 rounding:
    # the same codes, scales and bf16 side output as quantizing x.to(bfloat16), for the
    # vector and element paths, register-resident and streamed rows, the host seed and the
    # device seed; and the oracle on those bf16 values agrees on sampled rows.
    m, k = shape
    x = torch.randn(m, k, generator=gen(m + k)) * 1e-2
    x[0, 0] = 1.0 + 2.0 ** -9  # a tie that rounds to even
    col = torch.rand(k, generator=gen(7)) * 0.08 + 0.02
    xd = x.to(cuda)
    if strided:
        xd = torch.empty(m, k + 3, device=cuda)[:, :k]
        xd.copy_(x.to(cuda))
    cd = col.to(cuda)
    xb = xd.to(torch.bfloat16)
    side_a = torch.empty(m, k, dtype=torch.bfloat16, device=cuda)
    side_b = torch.empty(m, k, dtype=torch.bfloat16, device=cuda)
    qa, sa = ops().quantize_rows(xd, cd, True, 4242, x_bf16=side_a, round_bf16=True)
    qb, sb = ops().quantize_rows(xb, cd, True, 4242, x_bf16=side_b)
    assert torch.equal(qa, qb) and torch.equal(sa, sb) and torch.equal(side_a, side_b)
    slot = torch.tensor([4242], dtype=torch.int64, device=cuda)
    qd, sd = ops().quantize_rows(xd, cd, True, 0, slot, round_bf16=True)
    assert torch.equal(qd, qb) and torch.equal(sd, sb)
    qn, sn = ops().quantize_rows(xd, None, False, 0, round_bf16=True)
    qn_ref, sn_ref = ops().quantize_rows(xb)
    assert torch.equal(qn, qn_ref) and torch.equal(sn, sn_ref)
    qc, sc = qa.cpu().numpy(), sa.cpu().numpy()
    for r0 in (0, m // 2, m - 1):
        q_ref, s_ref = oquant.quantize_rows_sr(xb[r0:r0 + 1].float().cpu().numpy(),
                                               col.numpy(), 4242, row_start=r0)
        assert np.array_equal(qc[r0:r0 + 1], q_ref) and sc[r0] == s_ref[0]
    q_abi = torch.empty(m, k, dtype=torch.int8, device=cuda)
    s_abi = torch.empty(m, device=cuda)
    nat.call("rk_quantize_rows", xd.data_ptr(), nat.RK_F32_AS_BF16, m, k, xd.stride(0), 1,
             cd.data_ptr(), 1, 4242, 0, q_abi.data_ptr(), k, s_abi.data_ptr(), None, 0,
             nat.stream_handle(cuda))
    torch.cuda.synchronize()
    assert torch.equal(q_abi, qb) and torch.equal(s_abi, sb)


def test_quantize_columns_matches_transposed_rows(cuda):
    x = torch.randn(384, 200, generator=gen(13)) * 2.0
    q, s = quantize_columns(x.to(cuda))
    q_ref, s_ref = oquant.quantize_columns(x.numpy())
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(f32bits(s), f32bits(s_ref))


# ---------------------------------------------------------------------------
# int8 GEMM
# ---------------------------------------------------------------------------
# Covers the generic kernel (ragged K or N) and the 32x32x32 kernel in both block
# configurations: 128 x 128 tiles (small grids, K < 1024) and 256 x 256 tiles (K >= 1024
# with at least 256 of them: 4100 x 4136 has ragged last row and column tiles and an odd
# number of k-steps).
GEMM_SHAPES = [(67, 35, 53), (48, 40, 53), (1, 64, 1), (128, 128, 64), (130, 200, 129),
               (256, 384, 512), (1000, 1536, 512), (300, 200, 256), (129, 8, 128),
               (2500, 1032, 1024), (1, 16, 128), (4100, 4136, 1216)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_int8_gemm_nt_bit_exact(cuda, m, n, k):
    g = gen(m * 7 + n)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    ls = torch.rand(m, generator=g) + 0.01
    rs = torch.rand(n, generator=g) + 0.01
    out = int8_mm_nt(a.to(cuda), b.to(cuda), ls.to(cuda), rs.to(cuda))
    ref = ogemm.scaled_int8_mm(a.numpy(), b.numpy().T, ls.numpy(), rs.numpy())
    assert np.array_equal(bits16(out), ref)
    out1 = int8_mm_nt(a.to(cuda), b.to(cuda), ls.to(cuda), None, torch.float32)
    ref1 = ogemm.scaled_int8_mm(a.numpy(), b.numpy().T, ls.numpy(), None)
    assert np.array_equal(f32bits(out1), (ref1.astype(np.uint32) << 16))


@pytest.mark.parametrize("max_code", [1, 2, 3, 7])
@pytest.mark.parametrize("m,n,k", [(67, 53, 35), (512, 1536, 512), (257, 130, 192),
                                   (4100, 4104, 1088)])
def test_packed_gemm_bit_exact(cuda, m, n, k, max_code):
    packed, scale = synthetic_state(n, k, max_code, seed=m + n + k)
    code, _ = oupd.unpack(packed, max_code)
    q = torch.randint(-127, 128, (m, k), generator=gen(m), dtype=torch.int8)
    ls = torch.rand(m, generator=gen(m + 1)) * 0.05 + 1e-3
    out = packed_int8_mm(q.to(cuda), torch.from_numpy(packed).to(cuda), max_code,
                         ls.to(cuda), torch.from_numpy(scale).to(cuda))
    ref = ogemm.scaled_int8_mm(q.numpy(), code.T, ls.numpy(), scale)
    assert np.array_equal(bits16(out), ref)


# The forward GEMM with the residual added in its epilogue: the float32 output of the
# plain GEMM plus R, bit for bit, in both block configurations, with R aliasing the output.
@pytest.mark.parametrize("m,n,k", [(300, 200, 192), (4100, 4104, 1088)])
def test_packed_gemm_residual_equals_gemm_then_add(cuda, m, n, k):
    from local_ai_training.int8_matmul import packed_int8_mm_residual

    packed, scale = synthetic_state(n, k, 2, seed=m + k)
    q = torch.randint(-127, 128, (m, k), generator=gen(m), dtype=torch.int8).to(cuda)
    ls = (torch.rand(m, generator=gen(m + 1)) * 0.05 + 1e-3).to(cuda)
    pd, rs = torch.from_numpy(packed).to(cuda), torch.from_numpy(scale).to(cuda)
    r = torch.randn(m, n, generator=gen(m + 2)).to(cuda)
    want = r + packed_int8_mm(q, pd, 2, ls, rs, torch.float32)
    got = packed_int8_mm_residual(q, pd, 2, ls, rs, r)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))
    inplace = r.clone()
    packed_int8_mm_residual(q, pd, 2, ls, rs, inplace, out=inplace)
    assert torch.equal(inplace.view(torch.int32), want.view(torch.int32))


def test_residual_gemm_rejects_partial_overlap_of_residual_and_output(cuda):
    # R == C (same rows, same stride) is the in-place form; an R shifted by one row inside
    # C's storage would let one block overwrite rows another block still reads.
    m, n, k = 64, 128, 128
    packed, scale = synthetic_state(n, k, 2, seed=7)
    q = torch.randint(-127, 128, (m, k), generator=gen(7), dtype=torch.int8).to(cuda)
    ls = torch.full((m,), 1e-3, device=cuda)
    pd, rs = torch.from_numpy(packed).to(cuda), torch.from_numpy(scale).to(cuda)
    buf = torch.zeros(m + 1, n, device=cuda)
    args = (q.data_ptr(), k, pd.data_ptr(), k, 2, ls.data_ptr(), rs.data_ptr())
    with pytest.raises(nat.NativeError, match="overlaps"):
        nat.call("rk_int8_gemm_packed_residual", *args, buf[1:].data_ptr(), n,
                 buf[:m].data_ptr(), n, m, n, k, nat.stream_handle(cuda))
    with pytest.raises(nat.NativeError, match="overlaps"):  # same start, other stride
        nat.call("rk_int8_gemm_packed_residual", *args, buf.data_ptr(), n // 2,
                 buf.data_ptr(), n, m, n, k, nat.stream_handle(cuda))


# Decode-sized M (<= 16 tokens) takes the small-M kernel: 1B-model layer shapes (qkv 6144 x
# 2048, contract 2048 x 5632, lm_head 8192 x 2048), partial 16-row groups, M of 1..16.
SMALL_M_SHAPES = [(1, 6144, 2048), (16, 2048, 5632), (3, 136, 64), (16, 8, 64), (5, 1032, 1024),
                  (1, 8192, 2048), (11, 5632, 2048)]


@pytest.mark.parametrize("m,n,k", SMALL_M_SHAPES)
def test_small_m_int8_gemm_bit_exact(cuda, m, n, k):
    g = gen(m * 13 + n + k)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    ls = torch.rand(m, generator=g) * 1e-3 + 1e-5
    rs = torch.rand(n, generator=g) + 0.01
    out = int8_mm_nt(a.to(cuda), b.to(cuda), ls.to(cuda), rs.to(cuda))
    ref = ogemm.scaled_int8_mm(a.numpy(), b.numpy().T, ls.numpy(), rs.numpy())
    assert np.array_equal(bits16(out), ref)
    out1 = int8_mm_nt(a.to(cuda), b.to(cuda), ls.to(cuda), None, torch.float32)
    ref1 = ogemm.scaled_int8_mm(a.numpy(), b.numpy().T, ls.numpy(), None)
    assert np.array_equal(f32bits(out1), (ref1.astype(np.uint32) << 16))


@pytest.mark.parametrize("max_code", [2, 3])
@pytest.mark.parametrize("m,n,k", SMALL_M_SHAPES)
def test_small_m_packed_gemm_bit_exact(cuda, m, n, k, max_code):
    packed, scale = synthetic_state(n, k, max_code, seed=m + n + k + max_code)
    code, _ = oupd.unpack(packed, max_code)
    q = torch.randint(-127, 128, (m, k), generator=gen(m + k), dtype=torch.int8)
    ls = torch.rand(m, generator=gen(m + 1)) * 0.05 + 1e-3
    out = packed_int8_mm(q.to(cuda), torch.from_numpy(packed).to(cuda), max_code,
                         ls.to(cuda), torch.from_numpy(scale).to(cuda))
    ref = ogemm.scaled_int8_mm(q.numpy(), code.T, ls.numpy(), scale)
    assert np.array_equal(bits16(out), ref)


def test_forward_gemm_full_op_shape_bit_exact(cuda):
    # BASELINE op: M=16384 tokens, K=512, N=2048, quinary codes, scales U[0.02, 0.1].
    m, n, k, mc = 16384, 2048, 512, 2
    packed, scale = synthetic_state(n, k, mc, seed=2048, random_pressure=False)
    x = torch.randn(m, k, generator=gen(1)).to(torch.bfloat16)
    q, s = quantize_rows(x.to(cuda))
    out = packed_int8_mm(q, torch.from_numpy(packed).to(cuda), mc, s,
                         torch.from_numpy(scale).to(cuda))
    code, _ = oupd.unpack(packed, mc)
    ref = ogemm.scaled_int8_mm(q.cpu().numpy(), code.T, s.cpu().numpy(), scale)
    assert np.array_equal(bits16(out), ref)


@pytest.mark.parametrize("n,k", [(2048, 512), (1040, 528), (64, 48), (16, 16), (37, 45),
                                 (130, 64)])
@pytest.mark.parametrize("mc", [1, 2, 3, 7])
def test_unpack_transpose_matches_oracle(cuda, n, k, mc):
    # Aligned shapes (n, k multiples of 16) take the 16-byte decode/gather kernel, partial
    # 64 x 64 tiles included; the others the element-wise one.
    packed, _ = synthetic_state(n, k, mc, seed=n + k + mc)
    code_t = unpack_transpose(torch.from_numpy(packed).to(cuda), mc)
    code, _ = oupd.unpack(packed, mc)
    assert code_t.shape == (k, n)
    assert np.array_equal(code_t.cpu().numpy(), code.T)


def test_grad_input_gemm_full_op_shape_bit_exact(cuda):
    # int8 grad_input: A = SR-quantized gradient [M, N_out], B = code^T [K_in, N_out].
    m, n_out, k_in, mc = 16384, 2048, 512, 2
    packed, _ = synthetic_state(n_out, k_in, mc, seed=77)
    gq = torch.randint(-127, 128, (m, n_out), generator=gen(2), dtype=torch.int8)
    gs = torch.rand(m, generator=gen(3)) * 1e-3 + 1e-5
    code_t = unpack_transpose(torch.from_numpy(packed).to(cuda), mc)
    code, _ = oupd.unpack(packed, mc)
    assert np.array_equal(code_t.cpu().numpy(), code.T)
    out = int8_mm_nt(gq.to(cuda), code_t, gs.to(cuda), None, torch.float32)
    ref = ogemm.scaled_int8_mm(gq.numpy(), code, gs.numpy(), None)
    assert np.array_equal(f32bits(out), (ref.astype(np.uint32) << 16))


# The packed state as the [K, N] operand (grad_input contracts over the packed rows): tiles
# staged as they lie, transposed by ds_read_b64_tr_b8. Shapes: the op shape, partial 128-wide
# column tiles, small and ragged M, K of one k-step, every max_code.
PACKED_T_SHAPES = [(16384, 2048, 512), (300, 1024, 144), (1, 64, 16), (129, 192, 1040),
                   (77, 128, 2064), (4100, 1216, 4112)]


@pytest.mark.parametrize("m,k,n", PACKED_T_SHAPES)
@pytest.mark.parametrize("mc", [1, 3, 7])
def test_packed_t_gemm_matches_oracle(cuda, m, k, n, mc):
    from local_ai_training.int8_matmul import packed_int8_mm_t

    packed, scale = synthetic_state(k, n, mc, seed=m + k + n + mc)  # [K, N]
    code, _ = oupd.unpack(packed, mc)
    gq = torch.randint(-127, 128, (m, k), generator=gen(m + mc), dtype=torch.int8)
    gs = torch.rand(m, generator=gen(m + 7)) * 1e-3 + 1e-5
    out = packed_int8_mm_t(gq.to(cuda), torch.from_numpy(packed).to(cuda), mc, gs.to(cuda),
                           None, torch.float32)
    ref = ogemm.scaled_int8_mm(gq.numpy(), code, gs.numpy(), None)
    assert np.array_equal(f32bits(out), (ref.astype(np.uint32) << 16))
    if m <= 300:
        rs = (torch.rand(n, generator=gen(n)) + 0.01)
        out16 = packed_int8_mm_t(gq.to(cuda), torch.from_numpy(packed).to(cuda), mc,
                                 gs.to(cuda), rs.to(cuda))
        ref16 = ogemm.scaled_int8_mm(gq.numpy(), code, gs.numpy(), rs.numpy())
        assert np.array_equal(bits16(out16), ref16)


def test_packed_t_gemm_strided_rows_and_unsupported_shapes(cuda):
    from local_ai_training.int8_matmul import packed_int8_mm_t, packed_t_supported

    mc = 2
    packed, _ = synthetic_state(128, 96, mc, seed=5)
    code, _ = oupd.unpack(packed, mc)
    wide = torch.zeros(128, 160, dtype=torch.uint8)
    wide[:, :96] = torch.from_numpy(packed)
    p_view = wide.to(cuda)[:, :96]                      # ldp 160
    gq = torch.randint(-127, 128, (40, 144), generator=gen(9), dtype=torch.int8)
    a_view = gq.to(cuda)[:, :128]                       # lda 144
    gs = torch.rand(40, generator=gen(10)) * 1e-3 + 1e-5
    assert packed_t_supported(a_view, p_view)
    out = packed_int8_mm_t(a_view, p_view, mc, gs.to(cuda), None, torch.float32)
    ref = ogemm.scaled_int8_mm(gq[:, :128].numpy(), code, gs.numpy(), None)
    assert np.array_equal(f32bits(out), (ref.astype(np.uint32) << 16))
    ragged = torch.from_numpy(synthetic_state(100, 96, mc, seed=6)[0]).to(cuda)  # K % 64
    assert not packed_t_supported(gq.to(cuda)[:, :100], ragged)
    with pytest.raises(RuntimeError, match="K % 64"):
        packed_int8_mm_t(gq.to(cuda)[:, :100].contiguous(), ragged, mc, gs.to(cuda), None)


def test_scaled_int8_mm_public_api_strided_and_errors(cuda):
    # tests/test_int8_matmul.py:172-207
    g = gen(5)
    lhs = torch.randint(-20, 21, (48, 40), generator=g, dtype=torch.int8).to(cuda)
    weight = torch.randint(-8, 9, (53, 40), generator=g, dtype=torch.int8).to(cuda)
    ls = (torch.rand(48, generator=g) + 0.01).to(cuda)
    rs = (torch.rand(53, generator=g) + 0.01).to(cuda)
    strided = scaled_int8_mm(lhs, weight.t(), ls, rs)
    contiguous = scaled_int8_mm(lhs, weight.t().contiguous(), ls, rs)
    assert strided.dtype == torch.bfloat16 and torch.equal(strided, contiguous)
    expected = ((lhs.float() @ weight.t().float()) * ls[:, None] * rs[None, :]).to(torch.bfloat16)
    assert torch.equal(strided, expected)
    with pytest.raises(ValueError, match="finite and positive"):
        scaled_int8_mm(lhs, weight.t(), -ls, rs)
    with pytest.raises(TypeError):
        scaled_int8_mm(lhs.float(), weight.t(), ls, rs)
    with pytest.raises(ValueError, match="inner dimensions"):
        scaled_int8_mm(lhs, weight, ls, rs)


def test_effective_and_dequant_bf16_match_torch_formula(cuda):
    packed, scale = synthetic_state(53, 35, 3, seed=9)
    code, _ = oupd.unpack(packed, 3)
    eff = effective_bf16(torch.from_numpy(packed).to(cuda), 3, torch.from_numpy(scale).to(cuda))
    ref = torch.from_numpy(code).to(torch.bfloat16) * torch.from_numpy(scale).to(torch.bfloat16)[:, None]
    assert torch.equal(eff.cpu(), ref)
    q = torch.randint(-127, 128, (40, 32), generator=gen(8), dtype=torch.int8)
    s = torch.rand(40, generator=gen(9)) * 0.1
    xh = dequant_bf16(q.to(cuda), s.to(cuda))
    assert torch.equal(xh.cpu(), q.to(torch.bfloat16) * s[:, None].to(torch.bfloat16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 1), (63, 65), (64, 64), (130, 7), (257, 300),
                                   (16384, 2048)])
def test_transpose_bf16_is_rne_cast_then_transpose(cuda, shape, dtype):
    m, n = shape
    x = (torch.randn(m, n, generator=gen(m * 7 + n)) * 3).to(dtype)
    t = transpose_bf16(x.to(cuda))
    assert t.shape == (n, m) and t.is_contiguous()
    assert np.array_equal(bits16(t), bits16(x.to(torch.bfloat16).t().contiguous()))


def test_transpose_bf16_of_strided_rows(cuda):
    base = torch.randn(70, 96, generator=gen(5)).to(cuda)
    view = base[:, 8:72]
    t = transpose_bf16(view)
    assert np.array_equal(bits16(t), bits16(view.cpu().to(torch.bfloat16).t().contiguous()))


@pytest.mark.parametrize("shape", [(1, 64), (40, 32), (129, 257), (16384, 512)])
def test_dequant_transpose_matches_dequant_then_transpose(cuda, shape):
    m, k = shape
    q = torch.randint(-127, 128, (m, k), generator=gen(m + k), dtype=torch.int8)
    s = torch.rand(m, generator=gen(k)) * 0.1
    xt = dequant_transpose_bf16(q.to(cuda), s.to(cuda))
    ref = (q.to(torch.bfloat16) * s[:, None].to(torch.bfloat16)).t().contiguous()
    assert xt.shape == (k, m)
    assert np.array_equal(bits16(xt), bits16(ref))


# ---------------------------------------------------------------------------
# Ratchet update
# ---------------------------------------------------------------------------
def _update_z(packed: torch.Tensor, z: torch.Tensor, mc: int, T: int, low=0.5, high=1.5):
    counts = torch.zeros(4, dtype=torch.int64, device=packed.device)
    rows, k = z.shape
    nat.call("rk_ratchet_update", packed.data_ptr(), packed.stride(0), z.data_ptr(), k, rows, k,
             mc, T, low, high, counts.data_ptr(), nat.stream_handle(packed.device))
    return counts


@pytest.mark.parametrize("max_code,threshold", [(1, 1), (2, 2), (2, 8), (3, 4), (4, 8), (7, 3)])
@pytest.mark.parametrize("rows,k", [(6, 8), (48, 32), (37, 1001), (2048, 512)])
def test_update_from_normalized_gradient_bit_exact(cuda, rows, k, max_code, threshold):
    packed, _ = synthetic_state(rows, k, max_code, seed=rows * k + max_code)
    if threshold < 8:  # stored |pressure| < threshold for a reachable state
        _, p = oupd.unpack(packed, max_code)
        c, _ = oupd.unpack(packed, max_code)
        packed = oupd.pack(c, np.clip(p, -(threshold - 1), threshold - 1), max_code)
    z = torch.randn(rows, k, generator=gen(rows + k)) * 2.0
    pd = torch.from_numpy(packed).to(cuda)
    counts = _update_z(pd, z.to(cuda), max_code, threshold)
    ref, ref_counts = oupd.update_core(packed, z.numpy(), max_code, threshold)
    assert np.array_equal(pd.cpu().numpy(), ref)
    assert counts.cpu().tolist() == ref_counts.tolist()


def _update_grad(packed, g, mc, T, eps=1e-8, ema=None, beta=0.0, want_scale=True, low=0.5,
                 high=1.5):
    dev = packed.device
    rows, k = g.shape
    counts = torch.zeros(4, dtype=torch.int64, device=dev)
    row_rms = torch.empty(rows, device=dev)
    gscale = torch.empty(rows, device=dev) if want_scale else None
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    nat.call("rk_ratchet_update_grad", packed.data_ptr(), packed.stride(0), g.data_ptr(),
             nat.dtype_code(g.dtype), g.stride(0), rows, k, mc, T, low, high, eps, nat.ptr(ema),
             beta, 1.0 - beta, counts.data_ptr(), row_rms.data_ptr(), nat.ptr(gscale),
             flag.data_ptr(), None, nat.stream_handle(dev))
    return counts, row_rms, gscale, flag


@pytest.mark.parametrize("rows,k", [(6, 8), (37, 1001), (2048, 512), (8192, 512), (1, 64)])
def test_update_writes_the_mean_row_rms(cuda, rows, k):
    # rms_mean = mean of row_rms, summed in a fixed order: matches float64 and repeats
    # bit for bit.
    packed, _ = synthetic_state(rows, k, 2, seed=rows + k)
    g = torch.randn(rows, k, generator=gen(rows)).to(cuda) * 1e-2
    means = []
    for _ in range(3):
        pd = torch.from_numpy(packed).to(cuda)
        counts = torch.zeros(4, dtype=torch.int64, device=cuda)
        row_rms = torch.empty(rows, device=cuda)
        mean = torch.empty((), device=cuda)
        nat.call("rk_ratchet_update_grad", pd.data_ptr(), k, g.data_ptr(), nat.RK_F32, k, rows,
                 k, 2, 8, 0.5, 1.5, 1e-8, None, 0.0, 1.0, counts.data_ptr(),
                 row_rms.data_ptr(), None, None, mean.data_ptr(), nat.stream_handle(cuda))
        want = row_rms.double().mean().item()
        assert abs(mean.item() - want) <= 1e-6 * abs(want)
        means.append(mean.view(torch.int32).item())
    assert means[0] == means[1] == means[2]
    with pytest.raises(nat.NativeError, match="rms_mean needs row_rms"):
        nat.call("rk_ratchet_update_grad", pd.data_ptr(), k, g.data_ptr(), nat.RK_F32, k, rows,
                 k, 2, 8, 0.5, 1.5, 1e-8, None, 0.0, 1.0, counts.data_ptr(), None, None, None,
                 mean.data_ptr(), nat.stream_handle(cuda))
    # the same row rms as one segment among others of a shared buffer: rk_row_rms_means
    # gives the update's rms_mean bit for bit, every segment its own float64 mean, an
    # empty segment NaN
    other = torch.rand(3000, generator=gen(7)).to(cuda)
    buf = torch.cat([other[:1000], row_rms, torch.empty(0, device=cuda), other[1000:]])
    bounds = [0, 1000, 1000 + rows, 1000 + rows, buf.numel()]
    offsets = torch.tensor(bounds, dtype=torch.int64, device=cuda)
    seg = torch.empty(4, device=cuda)
    nat.call("rk_row_rms_means", buf.data_ptr(), buf.numel(), offsets.data_ptr(), 4,
             seg.data_ptr(), nat.stream_handle(cuda))
    assert seg[1].view(torch.int32).item() == means[0]
    for i in (0, 3):
        want = buf[bounds[i]:bounds[i + 1]].double().mean().item()
        assert abs(seg[i].item() - want) <= 1e-6 * abs(want)
    assert math.isnan(seg[2].item())
    # offsets past the buffer (or reversed, or negative) are clamped to [0, n]: the last
    # segment reads up to the end only, a segment wholly past the end is empty (NaN)
    n = buf.numel()
    bad = torch.tensor([1000, n + 5000, n + 9000, -7, 1000 + rows], dtype=torch.int64,
                       device=cuda)
    seg4 = torch.empty(4, device=cuda)
    nat.call("rk_row_rms_means", buf.data_ptr(), n, bad.data_ptr(), 4, seg4.data_ptr(),
             nat.stream_handle(cuda))
    want = buf[1000:].double().mean().item()
    assert abs(seg4[0].item() - want) <= 1e-6 * abs(want)
    assert math.isnan(seg4[1].item()) and math.isnan(seg4[2].item())
    want = buf[0:1000 + rows].double().mean().item()
    assert abs(seg4[3].item() - want) <= 1e-6 * abs(want)
    torch.cuda.synchronize()


# 4100 and 9000 rows take the pipelined row loop (several rows per wavefront, the next
# row's loads in flight during the current row's arithmetic): 9000 leaves wavefronts with
# two and with three rows, and every wavefront prefetches one row past the end.
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,k", [(6, 8), (37, 1001), (2048, 512), (512, 2048), (64, 5632),
                                    (16, 12000), (4100, 512), (9000, 256), (4099, 1000)])
def test_fused_normalize_update_bit_exact(cuda, rows, k, dtype):
    mc, T = 2, 8
    packed, _ = synthetic_state(rows, k, mc, seed=rows + 3 * k)
    g = (torch.randn(rows, k, generator=gen(rows * 5 + k)) * 1e-3).to(dtype)
    pd = torch.from_numpy(packed).to(cuda)
    counts, row_rms, gscale, flag = _update_grad(pd, g.to(cuda), mc, T)
    vec = oupd.vec_for_dtype("f32" if dtype == torch.float32 else "bf16")
    ref = oupd.update_from_gradient(packed, g.float().numpy(), mc, T, 0.5, 1.5, 1e-8, vec)
    assert np.array_equal(pd.cpu().numpy(), ref["packed"])
    assert counts.cpu().tolist() == ref["counts"].tolist()
    assert np.array_equal(f32bits(row_rms), f32bits(ref["row_rms"]))
    assert np.array_equal(f32bits(gscale), f32bits(ref["grad_scale"]))
    assert int(flag.item()) == 0


def _reduce_partials(part):
    """bf16(sum of the splits in order), the grad_weight reduction (IEEE float adds)."""
    acc = part[0].clone()
    for sp in range(1, part.shape[0]):
        acc = acc + part[sp]
    return acc.to(torch.bfloat16)


# The update fed by grad_weight's split partials (reduction fused into the update): every
# output equal to reducing to bf16 first and updating after. Shapes: the op shape, one
# chunk, several register chunks, streaming rows (K > 12 chunks), one split, many splits.
@pytest.mark.parametrize("rows,k,nsplit", [(2048, 512, 8), (96, 1024, 3), (64, 6144, 2),
                                           (33, 7168, 5), (8, 8, 1), (130, 2048, 17),
                                           (4100, 2048, 1), (9000, 512, 3)])
def test_update_from_partials_equals_reduce_then_update(cuda, rows, k, nsplit):
    mc, beta = 3, 0.9
    packed, _ = synthetic_state(rows, k, mc, seed=rows + k)
    part = torch.randn(nsplit, rows, k, generator=gen(rows * k)) * 1e-3
    part[:, 3 % rows, 1] = float("nan") if rows > 3 else 0.0  # a non-finite row is skipped
    part = part.to(cuda)
    gw = _reduce_partials(part)
    outs = []
    for fused in (False, True):
        pd = torch.from_numpy(packed).to(cuda)
        ema = torch.full((rows,), 0.25, device=cuda)
        counts = torch.zeros(4, dtype=torch.int64, device=cuda)
        row_rms = torch.empty(rows, device=cuda)
        gscale = torch.empty(rows, device=cuda)
        flag = torch.zeros(1, dtype=torch.int32, device=cuda)
        mean = torch.empty((), device=cuda)
        kept = torch.zeros(rows, k, dtype=torch.bfloat16, device=cuda)
        if fused:
            nat.call("rk_ratchet_update_partials", pd.data_ptr(), k, part.data_ptr(), nsplit,
                     rows, k, mc, 8, 0.5, 1.5, 1e-8, ema.data_ptr(), beta, 1.0 - beta,
                     counts.data_ptr(), row_rms.data_ptr(), gscale.data_ptr(),
                     flag.data_ptr(), mean.data_ptr(), kept.data_ptr(), k,
                     nat.stream_handle(cuda))
        else:
            nat.call("rk_ratchet_update_grad", pd.data_ptr(), k, gw.data_ptr(), nat.RK_BF16,
                     k, rows, k, mc, 8, 0.5, 1.5, 1e-8, ema.data_ptr(), beta, 1.0 - beta,
                     counts.data_ptr(), row_rms.data_ptr(), gscale.data_ptr(),
                     flag.data_ptr(), mean.data_ptr(), nat.stream_handle(cuda))
            kept = gw
        torch.cuda.synchronize()
        outs.append((pd, ema, counts, row_rms, gscale, flag, mean, kept))
    (pa, ea, ca, ra, ga, fa, ma, ka), (pb, eb, cb, rb, gb, fb, mb, kb) = outs
    assert torch.equal(pa, pb) and torch.equal(ca, cb) and torch.equal(fa, fb)
    finite = torch.isfinite(ra)
    for x, y in ((ea, eb), (ra, rb), (ga, gb)):
        assert torch.equal(x[finite].view(torch.int32), y[finite].view(torch.int32))
    assert torch.equal(ma.view(torch.int32), mb.view(torch.int32)) or bool(ma.isnan() & mb.isnan())
    ok = torch.isfinite(gw.float()).all(dim=1)
    assert torch.equal(ka[ok].view(torch.int16), kb[ok].view(torch.int16))
    if rows > 3:
        assert int(fb.item()) == 1


def test_grad_weight_partials_reduce_to_the_entry_point_result(cuda):
    # grad_weight with out = NULL leaves partials whose in-order sum, rounded to bf16, is
    # exactly what the entry point's own reduction writes
    m, n, k = 2048, 384, 512
    q = torch.randint(-127, 128, (m, k), generator=gen(41), dtype=torch.int8).to(cuda)
    s = (torch.rand(m, generator=gen(42)) * 0.05 + 1e-3).to(cuda)
    g = (torch.randn(m, n, generator=gen(43)) * 1e-2).to(torch.bfloat16).to(cuda)
    part = grad_weight_bf16(g, q, s, reduce=False)
    assert part.dtype == torch.float32 and part.shape[1:] == (n, k)
    want = grad_weight_bf16(g, q, s, part.shape[0])
    assert torch.equal(_reduce_partials(part).view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("shape,form", [
    (shape, form) for shape in [(2048, 384, 512), (4096, 1024, 1024), (1000, 264, 272)]
    for form in ("q8", "bf16", "f32")] + [((2048, 384, 512), "parts"),
                                          ((1000, 768, 1024), "parts")])
def test_one_split_gradient_written_directly_equals_the_reduced_partial(cuda, shape, form):
    # One split: the GEMM's epilogue writes the bf16 gradient itself (the entry point with
    # nsplit = 1, and the partials operators on a bf16 [1, N, K] work tensor). It equals
    # the split's float32 partial rounded by the reduction, bit for bit: the three
    # activation forms and a gradient in three column parts, both tile configurations
    # (1024 x 1024 takes the 256 x 256 tiles) and ragged tiles.
    m, n, k = shape
    q = torch.randint(-127, 128, (m, k), generator=gen(51), dtype=torch.int8).to(cuda)
    s = (torch.rand(m, generator=gen(52)) * 0.05 + 1e-3).to(cuda)
    g = (torch.randn(m, n, generator=gen(53)) * 1e-2).to(torch.bfloat16).to(cuda)
    x = (torch.randn(m, k, generator=gen(54))).to(cuda)
    f32 = torch.empty(1, n, k, device=cuda)
    direct = torch.empty(1, n, k, dtype=torch.bfloat16, device=cuda)
    if form == "q8":
        grad_weight_bf16(g, q, s, reduce=False, work=f32)
        grad_weight_bf16(g, q, s, reduce=False, work=direct)
        entry = grad_weight_bf16(g, q, s, 1)
    elif form == "parts":
        parts = list(g.chunk(3, dim=1))
        grad_weight_bf16_parts(parts, q, s, work=f32)
        grad_weight_bf16_parts(parts, q, s, work=direct)
        entry = grad_weight_bf16(g, q, s, 1)
    else:
        xx = x.to(torch.bfloat16) if form == "bf16" else x
        grad_weight_bf16_x(g, xx, reduce=False, work=f32)
        grad_weight_bf16_x(g, xx, reduce=False, work=direct)
        entry = grad_weight_bf16_x(g, xx, 1)
    want = _reduce_partials(f32)
    assert torch.equal(direct[0].view(torch.int16), want.view(torch.int16))
    assert torch.equal(entry.view(torch.int16), want.view(torch.int16))


def test_one_split_layer_update_equals_the_partials_update(cuda):
    # A layer whose grad_weight takes one split (4096 x 2048: 128 large tiles) hands the
    # update the bf16 gradient written by the GEMM; forcing the float32 partials path gives
    # the same state, counts, row rms and mean, over two steps.
    from local_ai_training import ratchet as ratchet_mod
    from local_ai_training.int8_matmul import grad_weight_splits, quantize_rows

    m, k, n = 4096, 2048, 4096
    assert grad_weight_splits(m, n, k) == 1
    outs = []
    for force_f32 in (False, True):
        torch.manual_seed(0)
        layer = ratchet_mod.DiscreteRatchetLinear(
            k, n, max_code=3, matmul_mode="int8", int8_backward=True,
            fuse_backward_update=True).to(cuda).train()
        layer.keep_weight_gradient = True
        # pressures one step short of the threshold, so the steps move codes
        near = (torch.randint(0, 2, (n, k), generator=gen(59), dtype=torch.int8) * 14 - 7)
        layer.packed.copy_(ratchet_mod.pack_code_pressure(layer.code.cpu(), near, 3).to(cuda))
        if force_f32:
            layer._split_workspace = lambda tokens, device: torch.empty(
                1, n, k, device=device, dtype=torch.float32)
        rec = []
        for step in range(2):
            x = torch.randn(m, k, generator=gen(60 + step)).to(torch.bfloat16).to(cuda)
            gout = (torch.randn(m, n, generator=gen(70 + step)) * 1e-2).to(torch.bfloat16)
            q, qs = quantize_rows(x)
            out = layer(x.requires_grad_(True), inputs_int8=q, inputs_scale=qs)
            torch.manual_seed(5 + step)
            out.backward(gout.to(cuda))
            st = layer.ratchet_update(validate=True)
            rec.append((layer.packed.clone(), [int(st.positive_moves), int(st.negative_moves),
                                               int(st.blocked_positive_moves),
                                               int(st.blocked_negative_moves)],
                        float(st.gradient_rms_mean), layer.last_weight_gradient.clone()))
        outs.append(rec)
    for (pa, ca, ra, ga), (pb, cb, rb, gb) in zip(*outs):
        assert torch.equal(pa, pb) and ca == cb and ra == rb
        assert torch.equal(ga.view(torch.int16), gb.view(torch.int16))
    assert sum(outs[0][0][1]) > 0


def test_fused_update_rms_ema_bit_exact(cuda):
    rows, k, mc, beta = 64, 512, 3, 0.9
    packed, _ = synthetic_state(rows, k, mc, seed=5)
    ema = np.zeros(rows, np.float32)
    pd = torch.from_numpy(packed).to(cuda)
    ema_d = torch.from_numpy(ema.copy()).to(cuda)
    for step in range(3):
        g = torch.randn(rows, k, generator=gen(step)) * (step + 1)
        if step == 2:
            g[5] = 0.0  # a row without gradient keeps its EMA
        _update_grad(pd, g.to(cuda), mc, 8, ema=ema_d, beta=beta, want_scale=False)
        ref = oupd.update_from_gradient(packed, g.numpy(), mc, 8, 0.5, 1.5, 1e-8, 4,
                                        rms_ema=ema, beta=beta)
        packed, ema = ref["packed"], ref["rms_ema"]
        assert np.array_equal(pd.cpu().numpy(), packed)
        assert np.array_equal(f32bits(ema_d), f32bits(ema))


def _smallest_reaching(c, d):
    """Smallest float32 t >= 0 whose float32 quotient t / d is >= c (brute-force walk)."""
    c, d = np.float32(c), np.float32(d)
    t = np.float32(c * d)
    while not np.float32(t / d) >= c:
        t = np.nextafter(t, np.float32(np.inf))
    while np.float32(np.nextafter(t, np.float32(0)) / d) >= c:
        t = np.nextafter(t, np.float32(0))
    return t


# The update buckets |g / d| against low / high; gradients placed on the exact float
# boundaries of those buckets (the boundary value, one ulp below, one ulp above, both
# signs) must bucket exactly as the division does. The row divisor d is pinned through
# the RMS EMA (beta 1: d = sqrt(ema) + eps, whatever the row holds); cases cover
# d from 1e-15 to 2e10, low == 0, and a subnormal d (eps 1e-39, rows too small to square).
@pytest.mark.parametrize("low,high,ema_val,eps", [
    (0.5, 1.5, 0.37, 1e-8), (1e-3, 2.0, 1e-30, 1e-30), (0.7, 0.9, 4e20, 1e-8),
    (0.5, 1.5, 1.0, 1e-12), (0.0, 1.5, 0.5, 1e-8), (0.25, 3.0, None, 1e-39)])
def test_fused_update_bucket_boundaries_bit_exact(cuda, low, high, ema_val, eps):
    rows, k, mc, T = 24, 512, 3, 3
    packed, _ = synthetic_state(rows, k, mc, seed=77)
    rng = np.random.default_rng(78)
    if ema_val is None:
        d = np.float32(eps)  # every g * g underflows: rms 0
        scale = d
    else:
        d = np.float32(np.sqrt(np.float32(ema_val))) + np.float32(eps)
        scale = d
    edges = []
    for c in (low, high):
        if c <= 0.0:
            continue
        t = _smallest_reaching(c, d)
        below = np.nextafter(t, np.float32(0))
        assert np.float32(t / d) >= np.float32(c) > np.float32(below / d)
        edges += [t, below, np.nextafter(t, np.float32(np.inf))]
    edges = np.array(edges + [0.0, 1e-45], np.float32)
    edges = np.concatenate([edges, -edges])
    g = (rng.standard_normal((rows, k)) * scale).astype(np.float32)
    for r in range(rows):
        cols = rng.choice(k, size=4 * edges.size, replace=False)
        g[r, cols] = np.tile(edges, 4)
    if ema_val is None:
        assert not np.any(g * g)
    pd = torch.from_numpy(packed).to(cuda)
    ema = None if ema_val is None else np.full(rows, ema_val, np.float32)
    ema_d = None if ema is None else torch.from_numpy(ema.copy()).to(cuda)
    beta = 0.0 if ema is None else 1.0
    counts, _, gscale, flag = _update_grad(pd, torch.from_numpy(g).to(cuda), mc, T, eps=eps,
                                           ema=ema_d, beta=beta, low=low, high=high)
    ref = oupd.update_from_gradient(packed, g, mc, T, low, high, eps, 4, rms_ema=ema, beta=beta)
    assert np.array_equal(pd.cpu().numpy(), ref["packed"])
    assert counts.cpu().tolist() == ref["counts"].tolist()
    assert np.array_equal(f32bits(gscale), f32bits(ref["grad_scale"]))
    assert int(flag.item()) == 0


def test_fused_update_nonfinite_rows_unchanged_and_flagged(cuda):
    rows, k, mc = 8, 256, 2
    packed, _ = synthetic_state(rows, k, mc, seed=6)
    g = torch.randn(rows, k, generator=gen(6))
    g[2, 17] = float("nan")
    g[5, 0] = float("inf")
    pd = torch.from_numpy(packed).to(cuda)
    counts, _, _, flag = _update_grad(pd, g.to(cuda), mc, 2)
    ref = oupd.update_from_gradient(packed, g.numpy(), mc, 2, 0.5, 1.5, 1e-8, 4)
    assert int(flag.item()) == 1 and ref["nonfinite"] == 1
    assert np.array_equal(pd.cpu().numpy(), ref["packed"])
    assert counts.cpu().tolist() == ref["counts"].tolist()


def test_normalize_rows_matches_oracle(cuda):
    g = torch.randn(100, 700, generator=gen(12)) * 3.0
    z = torch.empty(100, 700, device=cuda)
    gd = g.to(cuda)
    nat.call("rk_normalize_rows", gd.data_ptr(), nat.RK_F32, 700, 100, 700, 1e-8, None, 0.0,
             1.0, z.data_ptr(), 700, None, nat.stream_handle(gd.device))
    ref, _, _ = oupd.normalize_rows(g.numpy(), 1e-8, 4)
    assert np.array_equal(f32bits(z), f32bits(ref))


def test_unpack_leak_and_validate(cuda):
    packed, _ = synthetic_state(33, 65, 3, seed=4)
    pd = torch.from_numpy(packed).to(cuda)
    code = torch.empty(packed.shape, dtype=torch.int8, device=cuda)
    pres = torch.empty_like(code)
    nat.call("rk_unpack", pd.data_ptr(), pd.numel(), 3, code.data_ptr(), pres.data_ptr(),
             nat.stream_handle(pd.device))
    c_ref, p_ref = oupd.unpack(packed, 3)
    assert np.array_equal(code.cpu().numpy(), c_ref) and np.array_equal(pres.cpu().numpy(), p_ref)
    nat.call("rk_pressure_leak", pd.data_ptr(), pd.numel(), 3, nat.stream_handle(pd.device))
    assert np.array_equal(pd.cpu().numpy(), oupd.pressure_leak(packed, 3))
    flags = torch.zeros(3, dtype=torch.int32, device=cuda)
    scale = torch.tensor([0.5, float("nan")], device=cuda)
    bad = torch.tensor([0x0F, 0x00], dtype=torch.uint8, device=cuda)  # code 12 > 3; p = -7
    nat.call("rk_validate_state", bad.data_ptr(), 2, 3, scale.data_ptr(), 2, flags.data_ptr(),
             nat.stream_handle(bad.device))
    assert flags.cpu().tolist() == [1, 0, 1]


# ---------------------------------------------------------------------------
# BF16 grad_weight from int8 activations (TN product, no transposed copies)
# ---------------------------------------------------------------------------
def _xhat(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """bf16(bf16(q) * bf16(s)[:, None]) as float32 (ratchet.py:73-75)."""
    return round_to_bf16(q.astype(np.float32) * round_to_bf16(s.astype(np.float32))[:, None])


# (1000, 2056, 2048) and (4096, 2048, 2064) take the 256 x 256 output tiles (ragged last
# row / column tile, ragged token range, two or more splits); the others 128 x 128.
@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,n,k", [(4096, 256, 128), (1000, 136, 48), (16384, 2048, 512),
                                   (31, 8, 16), (1000, 2056, 2048), (4096, 2048, 2064)])
def test_grad_weight_bit_exact_when_every_sum_is_exact(cuda, m, n, k, gdtype):
    # g = small integers * 2^-4, q integers, s = 2^-7: every product and every partial sum
    # is exactly representable in fp32, so the result is order-free and must equal the
    # bf16 rounding of the exact float64 sum bit for bit (pins indexing and layouts).
    rng = np.random.default_rng(m + n + k)
    g = (rng.integers(-8, 9, size=(m, n)) / 16.0).astype(np.float32)
    q = rng.integers(-127, 128, size=(m, k)).astype(np.int8)
    s = np.full(m, 2.0**-7, np.float32)
    gd = torch.from_numpy(g).to(cuda).to(gdtype)
    out = grad_weight_bf16(gd, torch.from_numpy(q).to(cuda), torch.from_numpy(s).to(cuda))
    exact = g.astype(np.float64).T @ _xhat(q, s).astype(np.float64)
    assert np.array_equal(bits16(out), f32_to_bf16_bits(exact.astype(np.float32)))


@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_grad_weight_op_shape_within_tolerance_and_deterministic(cuda, gdtype):
    # Op shape: M=16384 tokens, N=2048, K=512; gradient N(0, 1e-2), activations N(0, 1)
    # quantized per token. Tolerance rel 1e-2 / abs 1e-3 against an fp32 product of the
    # same bf16 operands.
    m, n, k = 16384, 2048, 512
    g = (torch.randn(m, n, generator=gen(61)) * 1e-2).to(gdtype)
    x = torch.randn(m, k, generator=gen(62))
    q, s = quantize_rows(x.to(cuda))
    gd = g.to(cuda)
    out = grad_weight_bf16(gd, q, s)
    ref = gd.to(torch.bfloat16).float().t() @ torch.from_numpy(
        _xhat(q.cpu().numpy(), s.cpu().numpy())).to(cuda)
    err = (out.float() - ref).abs()
    assert bool((err <= 1e-3 + 1e-2 * ref.abs()).all()), float(err.max())
    again = grad_weight_bf16(gd, q, s)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    # the split count changes the summation grouping only within the tolerance
    one = grad_weight_bf16(gd, q, s, nsplit=1)
    assert bool(((one.float() - ref).abs() <= 1e-3 + 1e-2 * ref.abs()).all())


@pytest.mark.parametrize("m,n,k", [(4096, 256, 128), (1000, 136, 48), (31, 8, 16),
                                   (1000, 2056, 2048)])
@pytest.mark.parametrize("xdtype", [torch.float32, torch.bfloat16])
def test_grad_weight_x_bit_exact_when_every_sum_is_exact(cuda, m, n, k, xdtype):
    # Activations given directly: x = integers * 2^-6 (exact in bf16), g = integers / 16,
    # so every partial sum is exact and the result is the bf16 of the float64 sum.
    rng = np.random.default_rng(m * 3 + n + k)
    g = (rng.integers(-8, 9, size=(m, n)) / 16.0).astype(np.float32)
    x = (rng.integers(-127, 128, size=(m, k)) / 64.0).astype(np.float32)
    out = grad_weight_bf16_x(torch.from_numpy(g).to(cuda), torch.from_numpy(x).to(cuda).to(xdtype))
    exact = g.astype(np.float64).T @ x.astype(np.float64)
    assert np.array_equal(bits16(out), f32_to_bf16_bits(exact.astype(np.float32)))


@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_grad_weight_x_equals_the_int8_form_on_the_dequantized_copy(cuda, gdtype):
    # Same operands, same tiling and summation order: the int8-activation entry point and
    # the bf16-activation one on dequant_bf16(q, s) agree bit for bit at the op shape.
    m, n, k = 16384, 2048, 512
    g = (torch.randn(m, n, generator=gen(63)) * 1e-2).to(gdtype).to(cuda)
    q, s = quantize_rows(torch.randn(m, k, generator=gen(64)).to(cuda))
    fused = grad_weight_bf16(g, q, s)
    direct = grad_weight_bf16_x(g, dequant_bf16(q, s))
    assert torch.equal(fused.view(torch.int16), direct.view(torch.int16))


def test_grad_weight_x_rounds_float32_activations_to_nearest_even(cuda):
    # Float32 activations are rounded to bf16 while staging: identical to passing the
    # RNE-cast bf16 copy, for values that are not bf16-representable.
    m, n, k = 2048, 512, 256
    g = (torch.randn(m, n, generator=gen(65)) * 1e-2).to(cuda)
    x = torch.randn(m, k, generator=gen(66)).to(cuda)
    a = grad_weight_bf16_x(g, x)
    b = grad_weight_bf16_x(g, x.to(torch.bfloat16))
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    ref = g.to(torch.bfloat16).float().t() @ x.to(torch.bfloat16).float()
    assert bool(((a.float() - ref).abs() <= 1e-3 + 1e-2 * ref.abs()).all())


def test_grad_weight_rejects_unaligned_shapes(cuda):
    g = torch.randn(64, 12, device=cuda)
    q = torch.zeros(64, 16, dtype=torch.int8, device=cuda)
    s = torch.ones(64, device=cuda)
    with pytest.raises(RuntimeError, match="N % 8 == 0"):
        grad_weight_bf16(g, q, s)
