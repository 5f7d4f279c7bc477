"""The torch.ops.ratchet operators: registration, schemas and fake kernels (no GPU).

Every operator the op library defines is registered, mutating operators declare exactly
the arguments they write, and the fake kernels give the shapes and dtypes of the real
results on meta tensors (what torch.compile tracing and FakeTensorMode rely on). The GPU
behaviour of each operator is checked by tests/test_gpu_ops.py (torch.library.opcheck).
"""

from __future__ import annotations

import pytest
import torch

from local_ai_training import ops

MUTATED = {
    "packed_mm_accumulate": {"acc"},
    "grad_weight_partials": {"work"},
    "grad_weight_partials_x": {"work"},
    "grad_weight_partials_parts": {"work"},
    "update_from_z": {"packed", "counts"},
    "update_from_grad": {"packed", "rms_ema", "counts", "row_rms", "grad_scale", "nonfinite",
                         "rms_mean"},
    "update_from_partials": {"packed", "rms_ema", "counts", "row_rms", "grad_scale",
                             "nonfinite", "rms_mean", "grad_out"},
    "update_multi": {"written"},
    "normalize_rows": {"rms_ema"},
    "pressure_leak": {"packed"},
    "quantize_rows": {"x_bf16"},
}


@pytest.fixture(scope="module")
def R():
    return ops.ratchet()


def test_every_operator_is_registered_with_a_kernel_for_the_gpu(R):
    for name in ops.OPERATORS:
        op = getattr(R, name).default
        if name == "grad_weight_splits":
            continue  # a host-side query (catch-all kernel)
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CUDA"), name


@pytest.mark.parametrize("name", ops.OPERATORS)
def test_schema_declares_exactly_the_written_arguments(R, name):
    schema = getattr(R, name).default._schema
    written = {a.name for a in schema.arguments if a.alias_info and a.alias_info.is_write}
    assert written == MUTATED.get(name, set())
    if written:
        assert not schema.returns or name in ("quantize_rows", "normalize_rows",
                                              "rmsnorm_quantize",
                                              "gelu_quantize", "transpose_quantize")


def meta(*shape, dtype=torch.float32):
    return torch.empty(shape, dtype=dtype, device="meta")


def test_fake_kernels_give_result_shapes_on_meta_tensors(R):
    m, k, n = 96, 128, 256
    q, s = meta(m, k, dtype=torch.int8), meta(m)
    packed = meta(n, k, dtype=torch.uint8)
    x = meta(m, k, dtype=torch.bfloat16)
    qq, ss = R.quantize_rows(x)
    assert (qq.shape, qq.dtype, ss.shape, ss.dtype) == ((m, k), torch.int8, (m,), torch.float32)
    assert R.packed_mm(q, packed, 2, s, None, torch.float32).shape == (m, n)
    assert R.packed_mm(q, packed, 2, s, None, torch.bfloat16).dtype == torch.bfloat16
    assert R.packed_mm_residual(q, packed, 2, s, None, meta(m, n)).shape == (m, n)
    gq = meta(m, n, dtype=torch.int8)
    assert R.packed_mm_t(gq, packed, 2, s, None, torch.float32).shape == (m, k)
    assert R.int8_mm_nt(q, meta(n, k, dtype=torch.int8), s, None, torch.bfloat16).shape == (m, n)
    assert R.unpack_transpose(packed, 2).shape == (k, n)
    code, pressure = R.unpack(packed, 2)
    assert code.shape == pressure.shape == (n, k) and code.dtype == torch.int8
    assert R.effective_bf16(packed, 2, meta(n)).shape == (n, k)
    assert R.dequant_bf16(q, s).shape == (m, k)
    assert R.transpose_bf16(x).shape == (k, m)
    assert R.dequant_transpose_bf16(q, s).shape == (k, m)
    g = meta(m, n, dtype=torch.bfloat16)
    gw = R.grad_weight(g, q, s)
    assert gw.shape == (n, k) and gw.dtype == torch.bfloat16
    assert R.grad_weight_x(g, x).shape == (n, k)
    assert R.normalize_rows(meta(n, k), 1e-8, None, 0.0).shape == (n, k)
    flags = R.validate_state(packed, 2, None)
    assert flags.shape == (3,) and flags.dtype == torch.int32
    for fn in (R.gelu_quantize,):
        a, b = fn(x)
        assert a.shape == (m, k) and b.shape == (m,)
    a, b = R.rmsnorm_quantize(x, meta(k), 1e-5)
    assert a.shape == (m, k) and b.shape == (m,)
    a, b = R.transpose_quantize(meta(2, 4, 48, 32, dtype=torch.bfloat16))
    assert a.shape == (96, 128) and b.shape == (96,)
    gx, gwn = R.rmsnorm_backward(x, x, meta(k), 1e-5)
    assert gx.shape == (m, k) and gx.dtype == torch.bfloat16 and gwn.dtype == torch.float32
    assert R.gelu_backward(meta(m, k), meta(m, k)).dtype == torch.float32
    emb = R.embedding_backward(meta(2, m // 2, k, dtype=torch.bfloat16),
                               meta(2, m // 2, dtype=torch.int64), 50)
    assert emb.shape == (50, k) and emb.dtype == torch.float32
    parts = [meta(m, n, dtype=torch.bfloat16) for _ in range(3)]
    qp, sp = R.quantize_rows_parts(parts, meta(3 * n), True, 7)
    assert (qp.shape, qp.dtype, sp.shape, sp.dtype) == ((m, 3 * n), torch.int8, (m,),
                                                          torch.float32)
    assert R.row_rms_means(meta(n), meta(5, dtype=torch.int64)).shape == (4,)
    ao, alse = R.attention_forward(*(meta(2, 3, 40, 64, dtype=torch.bfloat16) for _ in range(3)),
                                   0.125)
    assert ao.shape == (2, 3, 40, 64) and ao.stride() == (7680, 64, 192, 1)
    assert alse.shape == (2, 3, 40) and alse.dtype == torch.float32
    tg = meta(m, dtype=torch.int64)
    loss, stats, count = R.cross_entropy_forward(x, tg)
    assert (loss.shape, stats.shape, count.shape) == ((), (3, m), ())
    assert loss.dtype == stats.dtype == count.dtype == torch.float32
    grad = R.cross_entropy_backward(meta(), x, tg, stats, count)
    assert grad.shape == (m, k) and grad.dtype == torch.bfloat16


def test_split_count_query_runs_on_the_host(R):
    assert R.grad_weight_splits(16384, 2048, 512) >= 1
    assert R.grad_weight_splits(0, 1, 1) == 1


def test_operators_reject_cpu_tensors(R):
    with pytest.raises(NotImplementedError):
        R.packed_mm(torch.zeros(2, 64, dtype=torch.int8), torch.zeros(8, 64, dtype=torch.uint8),
                    2, torch.ones(2), None, torch.bfloat16)
